"""Pin the numpy oracle against closed forms, big-int brute force and the reference's own KATs (CPU only)."""
import math

import numpy as np
import pytest

from oracle import fixedpoint as fx
from oracle import prng
from oracle.q1 import q1_linear, q1_linear_bigint, unpack_signs
from oracle.rope import apply_neox, build_yarn_rope_tables

I64_MIN, I64_MAX = -(1 << 63), (1 << 63) - 1


def test_splitmix64_published_vector():
    # SplitMix64 seeded with 1234567 (Vigna's reference implementation, first three outputs)
    out = prng.splitmix64(1234567, 3)
    assert [int(v) for v in out] == [6457827717110365317, 3203168211198807973, 9817491932198370423]


def test_numpy_shift_semantics_the_oracle_relies_on():
    a = np.array([5, -5, 5, -5], dtype=np.int64)
    assert list(fx.rshift(a, np.array([-1, -1, 70, 70]))) == [0, -1, 0, -1]
    # plain numpy agrees for in-range counts (arithmetic = floor)
    assert list(a >> np.int64(1)) == [2, -3, 2, -3]


def test_q1_wrap_kat_from_reference_smoke_test():
    # bonsai/tests/test_bonsai_smoke.py:890-906: x[0,0]=2^62, bit0 set, frac=1, scales [3,-3,4].
    # S = 2^62; 3*2^62 = -2^62 (mod 2^64) -> >>1 = -2^61; -3*2^62 = 2^62 -> 2^61; 4*2^62 = 0.
    x = np.zeros((1, 128), dtype=np.int64)
    x[0, 0] = 1 << 62
    bits = np.zeros((3, 1, 16), dtype=np.uint8)
    bits[:, 0, 0] = 1
    scale = np.array([[3], [-3], [4]], dtype=np.int64)
    want = [-(1 << 61), 1 << 61, 0]
    assert list(q1_linear(x, bits, scale, 1)[0]) == want
    assert list(q1_linear_bigint(x, bits, scale, 1)[0]) == want


@pytest.mark.parametrize("frac", [0, 1, 16, 31, 62, 63])
def test_q1_expanded_matches_bigint_bruteforce(frac):
    rng = np.random.default_rng(frac + 7)
    N, nb, T = 5, 2, 2
    bits = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    scale = rng.integers(-(1 << 40), 1 << 40, size=(N, nb), dtype=np.int64)
    scale[0, 0] = I64_MIN
    scale[1, 1] = I64_MAX
    x = rng.integers(-(1 << 62), 1 << 62, size=(T, nb * 128), dtype=np.int64)
    x[0, :3] = [I64_MIN, I64_MAX, -1]
    assert np.array_equal(q1_linear(x, bits, scale, frac), q1_linear_bigint(x, bits, scale, frac))


def test_q1_bit_order_is_little_endian_per_byte():
    bits = np.zeros((1, 1, 16), dtype=np.uint8)
    bits[0, 0, 1] = 0b00000100          # weight 8*1 + 2 = 10 is +1, the rest -1
    s = unpack_signs(bits)[0, 0]
    assert s[10] == 1 and (s == -1).sum() == 127
    x = np.zeros((1, 128), dtype=np.int64)
    x[0, 10] = 7
    x[0, 11] = 100
    # S = 7 - 100 = -93; scale 2, frac 0
    assert q1_linear(x, bits, np.array([[2]]), 0)[0, 0] == -186


def test_q1_two_pos_minus_total_identity():
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 256, size=(4, 3, 16), dtype=np.uint8)
    x = rng.integers(-1000, 1000, size=(1, 384), dtype=np.int64)
    signs = unpack_signs(bits).astype(np.int64).reshape(4, 384)
    pos = ((signs > 0) * x).reshape(4, 3, 128).sum(-1)
    total = x.reshape(3, 128).sum(-1)
    direct = (signs * x).reshape(4, 3, 128).sum(-1)
    assert np.array_equal(2 * pos - total, direct)


def test_yarn_rope_kat_rows():
    # bonsai/tests/test_bonsai_smoke.py:91-107
    cos, sin = build_yarn_rope_tables(2, 128, base=1_000_000, freq_scale=0.25, n_ctx_orig=16_384)
    assert (int(cos[0, 0]), int(sin[0, 0])) == (74_621, 0)
    assert (int(cos[1, 0]), int(sin[1, 0])) == (40_318, 62_792)
    assert (int(cos[1, 10]), int(sin[1, 10])) == (74_124, 8_598)
    assert (int(cos[1, 19]), int(sin[1, 19])) == (74_611, 1_235)


def test_rope_neox_pairs_halves():
    cos = np.array([[0, 1 << 16]], dtype=np.int64)   # pair 0: 90 degrees, pair 1: identity (cos=1, sin=0)
    sin = np.array([[1 << 16, 0]], dtype=np.int64)
    x = np.array([[[3, 5, 7, 11]]], dtype=np.int64)   # halves (3,5) and (7,11): pairs (3,7) and (5,11)
    out = apply_neox(x, cos, sin, 16)[0, 0]
    assert list(out) == [-7, 5, 3, 11]


def test_exp2_integer_exponents_are_exact_powers():
    f = 16
    u = np.array([k << f for k in range(0, 20)], dtype=np.int64)
    assert list(fx.exp2_neg_fixed(u, f)) == [(1 << 16) >> k for k in range(20)]


def test_sigmoid_equals_two_logit_softmax():
    # bonsai/tests/test_bonsai_smoke.py:468-484
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.integers(-(1 << 22), 1 << 22, size=200), [0, 1, -1, 1 << 40, -(1 << 40)]]).astype(np.int64)
    sm = fx.softmax_rows(np.stack([np.zeros_like(x), x], axis=1), 16)[:, 1]
    assert np.array_equal(fx.sigmoid(x, 16), sm)


def test_silu_wraps_at_int64_extremes():
    x = np.array([I64_MIN, I64_MAX, I64_MIN + 1, 0], dtype=np.int64)
    out = fx.silu_wrap(x, 16)
    assert out[0] == 0 and out[3] == 0          # INT64_MIN * 2^15 wraps to 0 (worked in the module notes)


def test_rmsnorm_matches_isqrt_bigint():
    rng = np.random.default_rng(9)
    for mag in (14, 25, 40, 62):
        x = rng.integers(-(1 << mag), 1 << mag, size=(3, 64), dtype=np.int64)
        got = fx.rmsnorm(x, 16, 1)
        for r in range(3):
            ssq = sum(int(v) * int(v) for v in x[r])
            rms = math.isqrt(ssq // 64 + 1)
            assert [int(v) for v in got[r]] == [(int(v) << 16) // rms for v in x[r]]


def test_rmsnorm_gain_envelope_raises():
    x = np.array([[1 << 20, -(1 << 20)]], dtype=np.int64)
    with pytest.raises(OverflowError):
        fx.rmsnorm(x, 16, 1, np.array([1 << 60, 1], dtype=np.int64))


def test_attention_bound_raises_like_reference():
    q = np.full((1, 1, 8), 1 << 40, dtype=np.int64)
    with pytest.raises(OverflowError):
        fx.fixed_point_matmul(q[0], np.full((8, 1), 1 << 40, dtype=np.int64), 16)
