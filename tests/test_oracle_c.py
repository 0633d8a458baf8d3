"""The C restatement (oracle/c) equals the numpy oracle, and both equal the compiled reference C kernels
(oracle/_ref, built from /root/reference sources when present) — CPU only."""
import ctypes
from pathlib import Path

import numpy as np
import pytest

from oracle import c_oracle, fixedpoint as fx, prng
from oracle.attention import attention_cached
from oracle.q1 import q1_linear

REF = Path(__file__).resolve().parents[1] / "oracle" / "_ref"
I64_MIN, I64_MAX = -(1 << 63), (1 << 63) - 1


def _ref(name):
    p = REF / name
    if not p.exists():
        pytest.skip(f"{p} not built (needs /root/reference)")
    return ctypes.CDLL(str(p))


@pytest.mark.parametrize("T,N,nb,xmag,frac", [(1, 64, 4, 20, 16), (3, 40, 2, 62, 16), (9, 17, 3, 30, 0), (2, 8, 1, 63, 63)])
def test_c_q1_equals_numpy(T, N, nb, xmag, frac):
    rng = np.random.default_rng(T * 7 + N)
    bits = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    scale = rng.integers(I64_MIN, I64_MAX, size=(N, nb), dtype=np.int64)
    lo = I64_MIN if xmag == 63 else -(1 << xmag)
    hi = I64_MAX if xmag == 63 else (1 << xmag)
    x = rng.integers(lo, hi, size=(T, nb * 128), dtype=np.int64)
    assert np.array_equal(c_oracle.q1_linear(x, bits, scale, frac), q1_linear(x, bits, scale, frac))


def test_numpy_q1_equals_reference_c_kernel():
    so = _ref("libbonsai_q1_kernel.so")
    f = so.bonsai_q1_linear_i64
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 4 + [ctypes.c_void_p]
    rng = np.random.default_rng(4)
    for xmag, frac in ((20, 16), (62, 1), (40, 31)):
        bits = rng.integers(0, 256, size=(33, 5, 16), dtype=np.uint8)
        scale = rng.integers(-(1 << 40), 1 << 40, size=(33, 5), dtype=np.int64)
        x = rng.integers(-(1 << xmag), 1 << xmag, size=(2, 640), dtype=np.int64)
        out = np.empty((2, 33), dtype=np.int64)
        assert f(x.ctypes.data, bits.ctypes.data, scale.ctypes.data, 2, 33, 5, frac, out.ctypes.data) == 0
        assert np.array_equal(out, q1_linear(x, bits, scale, frac))


@pytest.mark.parametrize("mag", [10, 25, 40, 62])
def test_c_rmsnorm_equals_numpy(mag):
    rng = np.random.default_rng(mag)
    x = rng.integers(-(1 << mag), 1 << mag, size=(5, 96), dtype=np.int64)
    g = rng.integers(1 << 15, 1 << 17, size=96, dtype=np.int64)
    assert np.array_equal(c_oracle.rmsnorm(x, 16, 1, None), fx.rmsnorm(x, 16, 1, None))
    if mag < 40:
        assert np.array_equal(c_oracle.rmsnorm(x, 16, 1, g), fx.rmsnorm(x, 16, 1, g))


def test_numpy_rmsnorm_equals_reference_c_kernel():
    so = _ref("libbonsai_q1_kernel.so")
    f = so.bonsai_rmsnorm_i64
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] + [ctypes.c_int64] * 4 + [ctypes.c_void_p] * 2
    rng = np.random.default_rng(12)
    for mag in (14, 25, 40):
        x = rng.integers(-(1 << mag), 1 << mag, size=(4, 128), dtype=np.int64)
        g = rng.integers(1 << 14, 1 << 18, size=128, dtype=np.int64)
        out = np.empty_like(x)
        assert f(x.ctypes.data, 4, 128, 16, 1, g.ctypes.data, out.ctypes.data) == 0
        assert np.array_equal(out, fx.rmsnorm(x, 16, 1, g))


@pytest.mark.parametrize("H,Hkv,hd,M,start", [(4, 2, 32, 5, 0), (8, 2, 16, 1, 40), (4, 4, 8, 7, 3)])
def test_c_attention_equals_numpy(H, Hkv, hd, M, start):
    rng = np.random.default_rng(H * 31 + M)
    L = start + M
    q = rng.integers(-(1 << 20), 1 << 20, size=(H, M, hd), dtype=np.int64)
    k = rng.integers(-(1 << 20), 1 << 20, size=(Hkv, L, hd), dtype=np.int64)
    v = rng.integers(-(1 << 20), 1 << 20, size=(Hkv, L, hd), dtype=np.int64)
    assert np.array_equal(c_oracle.attention_cached(q, k, v, start, 16, 5793),
                          attention_cached(q, k, v, start, 16, 5793))


def test_numpy_attention_equals_reference_c_kernels():
    so = _ref("libbonsai_q1_kernel.so")
    dec = so.bonsai_attention_decode_i64
    dec.restype = ctypes.c_int
    dec.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 8 + [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    pre = so.bonsai_attention_prefill_i64
    pre.restype = ctypes.c_int
    pre.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 8 + [ctypes.c_void_p]
    rng = np.random.default_rng(77)
    H, Hkv, hd, L = 8, 2, 32, 57
    q = rng.integers(-(1 << 20), 1 << 20, size=(H, 1, hd), dtype=np.int64)
    k = rng.integers(-(1 << 20), 1 << 20, size=(Hkv, L, hd), dtype=np.int64)
    v = rng.integers(-(1 << 20), 1 << 20, size=(Hkv, L, hd), dtype=np.int64)
    out = np.empty((H, hd), dtype=np.int64)
    scratch = np.empty(H * L, dtype=np.int64)
    assert dec(q.ctypes.data, k.ctypes.data, v.ctypes.data, H, Hkv, hd, L, L * hd, L * hd, 16, 5793,
               out.ctypes.data, scratch.ctypes.data, scratch.size) == 0
    assert np.array_equal(out, attention_cached(q, k, v, L - 1, 16, 5793)[:, 0])
    M = 9
    qp = rng.integers(-(1 << 20), 1 << 20, size=(H, M, hd), dtype=np.int64)
    kp, vp = k[:, :M].copy(), v[:, :M].copy()
    outp = np.empty((H, M, hd), dtype=np.int64)
    assert pre(qp.ctypes.data, kp.ctypes.data, vp.ctypes.data, H, Hkv, hd, M, M, 0, 16, 5793, outp.ctypes.data) == 0
    assert np.array_equal(outp, attention_cached(qp, kp, vp, 0, 16, 5793))


def _silu_inputs(seed, n=4000):
    rng = np.random.default_rng(seed)
    x = np.concatenate([rng.integers(-(1 << 24), 1 << 24, size=n), rng.integers(I64_MIN, I64_MAX, size=64),
                        [0, 1, -1, I64_MIN, I64_MAX, I64_MIN + 1, 1 << 40, -(1 << 40)]]).astype(np.int64)
    up = rng.integers(-(1 << 30), 1 << 30, size=x.size).astype(np.int64)
    up[-8:] = [I64_MAX, I64_MIN, 3, -3, 1 << 62, -(1 << 62), 7, I64_MIN + 1]
    return x, up


@pytest.mark.parametrize("frac", [16, 1, 29])
def test_c_silu_mul_equals_numpy(frac):
    x, up = _silu_inputs(frac)
    want = fx.mulshift_wrap(fx.silu_wrap(x, frac), up, frac)
    assert np.array_equal(c_oracle.silu_mul(x, up, frac), want)


def test_c_silu_mul_equals_reference_c_kernel():
    """bonsai_q1_kernel.c:1729-1767 bonsai_silu_i64, then the mulshift of reference_bonsai.py:614."""
    so = _ref("libbonsai_q1_kernel.so")
    f = so.bonsai_silu_i64
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
    x, up = _silu_inputs(3)
    s = np.empty_like(x)
    assert f(x.ctypes.data, x.size, 16, s.ctypes.data) == 0
    assert np.array_equal(c_oracle.silu_mul(x, up, 16), fx.mulshift_wrap(s, up, 16))


@pytest.mark.parametrize("H,Hkv,hd,M,start,extra", [(4, 2, 32, 1, 40, 9), (8, 2, 16, 3, 5, 1), (2, 1, 128, 1, 0, 64)])
def test_c_attention_ld_equals_numpy_on_row_buffers(H, Hkv, hd, M, start, extra):
    """Rows [0, L) of (Hkv, L + extra, hd) buffers give the contiguous attention's result (decode over a cache
    with room for more rows)."""
    L = start + M
    rng = np.random.default_rng(H * 100 + L)
    q = rng.integers(-(1 << 20), 1 << 20, size=(H, M, hd), dtype=np.int64)
    kb = rng.integers(-(1 << 20), 1 << 20, size=(Hkv, L + extra, hd), dtype=np.int64)
    vb = rng.integers(-(1 << 20), 1 << 20, size=(Hkv, L + extra, hd), dtype=np.int64)
    kb[:, L:] = 1 << 40                                       # rows past L must not be read (bounds included)
    vb[:, L:] = -(1 << 40)
    want = attention_cached(q, kb[:, :L].copy(), vb[:, :L].copy(), start, 16, 5793)
    assert np.array_equal(c_oracle.attention_ld(q, kb, vb, L, start, 16, 5793), want)


def test_c_uniform_fill_equals_prng_stream():
    from oracle import workloads
    out = np.full((2 * 50, 40), 7, dtype=np.int64)
    c_oracle.uniform_fill(13, 100000 + 1024 * 3 + 512 + 5, out, 2 * 37, 32, -(1 << 20), 1 << 20)
    want = workloads.kv_fill_seq(13, 3, 1, 5, 2, 37, 32)
    assert np.array_equal(out[:74, :32], want.reshape(74, 32)) and (out[:74, 32:] == 7).all()
    assert (out[74:] == 7).all()
    part = np.zeros((37, 32), dtype=np.int64)                 # kv head 1 alone: stream offset 37 * 32
    c_oracle.uniform_fill(13, 100000 + 1024 * 3 + 512 + 5, part, 37, 32, -(1 << 20), 1 << 20, first=37 * 32)
    assert np.array_equal(part, want[1])
    big = np.empty((3, 5), dtype=np.int64)
    c_oracle.uniform_fill(2, 9, big, 3, 5, -(1 << 61), 1 << 62)
    assert np.array_equal(big, prng.uniform_int(2, 9, (3, 5), -(1 << 61), 1 << 62))
