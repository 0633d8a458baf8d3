"""Q1_0 linear on gfx950 vs the oracle, byte for byte (parity gates after bonsai/tests/test_bonsai_gpu.py:74-140)."""
import ctypes

import numpy as np
import pytest

from oracle import prng
from oracle.q1 import q1_linear, q1_linear_bigint

pytestmark = pytest.mark.gpu
I64_MIN, I64_MAX = -(1 << 63), (1 << 63) - 1


def test_mfma_operand_and_accumulator_layout(gpu):
    """Pin the v_mfma_i32_16x16x64_i8 lane mapping the Q1 kernels assume: A lane l = row l%16, B lane l =
    column l%16, both with K-group l//16 paired byte-for-byte; D lane l holds rows 4*(l//16)+r of column l%16."""
    from integer_inference_engine_amd import _lib
    so = _lib.lib()

    def run(a, b):
        d = np.zeros((64, 4), dtype=np.int32)
        assert so.imie_probe_mfma(a.ctypes.data, b.ctypes.data, d.ctypes.data) == 0
        return d

    rng = np.random.default_rng(1)
    a = rng.integers(-128, 128, size=(64, 16), dtype=np.int8)
    b = rng.integers(-128, 128, size=(64, 16), dtype=np.int8)
    d = run(a, b)
    A = np.zeros((16, 4, 16), dtype=np.int64)
    B = np.zeros((4, 16, 16), dtype=np.int64)
    for l in range(64):
        A[l % 16, l // 16] = a[l]
        B[l // 16, :, l % 16] = b[l]
    full = np.einsum("mgk,gkn->mn", A, B)
    for l in range(64):
        for r in range(4):
            assert d[l, r] == full[4 * (l // 16) + r, l % 16]


def test_mfma_peak_calibration_is_plausible(gpu):
    """The measured sustained int8 MFMA rate the bench quotes utilisation against: between 1 POPS and the published
    dense 5.0 POPS (plus clock headroom)."""
    from integer_inference_engine_amd import _lib
    so = _lib.lib()
    v = ctypes.c_double()
    assert so.imie_mfma_peak(ctypes.byref(v)) == 0
    assert 1.0e15 < v.value < 5.6e15


def test_hbm_read_peak_calibration_is_plausible(gpu):
    """The measured sustained HBM read rate the bench quotes the matvec against: between 2 TB/s and the published
    8 TB/s."""
    from integer_inference_engine_amd import _lib
    so = _lib.lib()
    v = ctypes.c_double()
    assert so.imie_hbm_read_peak(1 << 28, ctypes.byref(v)) == 0
    assert 2.0e12 < v.value < 8.0e12
    assert so.imie_hbm_read_peak(1 << 20, ctypes.byref(v)) != 0          # below the 16 MiB minimum: refused


@pytest.mark.parametrize("N,nb,T", [(16, 4, 1), (37, 3, 1), (256, 32, 1), (1024, 96, 1), (100, 5, 3), (64, 8, 7),
                                    # decode-sized launches whose waves request 4 / 2 slabs at once, with a short
                                    # last slab range (10 = 4 + 4 + 2 slabs, 25 = 12 * 2 + 1)
                                    (24576, 40, 1), (24576, 32, 1), (4096, 100, 1)])
def test_q1_apply_matches_oracle_shapes(gpu, N, nb, T):
    seed = N * 1000 + nb * 10 + T
    bits = prng.uniform_bytes(seed, 1, (N, nb, 16))
    scale = prng.uniform_int(seed, 2, (N, nb), -(1 << 11), 1 << 11)
    x = prng.uniform_int(seed, 3, (T, nb * 128), -(1 << 20), 1 << 20)
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None
    assert np.array_equal(got, q1_linear(x, bits, scale, 16))


@pytest.mark.parametrize("N,nb,T,xmag", [
    (64, 200, 3, 45),      # 50 slabs over 8 K-splits x 3 tokens: no staged limbs, every limb group from memory
    (64, 128, 4, 45),      # 16 staged slab-tokens: limbs 0-3 from LDS, limbs 4-7 from memory
    (64, 128, 4, 62),
    (24576, 40, 1, 45),    # decode launch, 4 slabs requested at once, two limb groups
    (4096, 100, 1, 62),    # decode launch, 2 slabs at once, eight limbs
])
def test_q1_limb_groups_from_lds_and_memory(gpu, N, nb, T, xmag):
    seed = N + nb + T + xmag
    bits = prng.uniform_bytes(seed, 1, (N, nb, 16))
    scale = prng.uniform_int(seed, 2, (N, nb), -(1 << 12), 1 << 12)
    x = prng.uniform_int(seed, 3, (T, nb * 128), -(1 << xmag), 1 << xmag)
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, q1_linear(x, bits, scale, 16))


@pytest.mark.parametrize("N,nb,T", [(4096, 32, 1), (24576, 40, 1), (64, 128, 4), (96, 24, 2)])
def test_q1_mixed_single_and_multi_limb_slabs(gpu, N, nb, T):
    # slabs alternate between |x| <= 127 (one limb: the bit-position row layout) and wide values (limb groups)
    seed = 7 * N + nb + T
    bits = prng.uniform_bytes(seed, 1, (N, nb, 16))
    scale = prng.uniform_int(seed, 2, (N, nb), -(1 << 20), 1 << 20)
    x = prng.uniform_int(seed, 3, (T, nb * 128), -127, 128)
    wide = prng.uniform_int(seed, 4, (T, nb * 128), -(1 << 40), 1 << 40)
    for sl in range(1, (nb + 3) // 4, 2):
        x[:, sl * 512:(sl + 1) * 512] = wide[:, sl * 512:(sl + 1) * 512]
    x[:, -1] = -128                                   # the one value that needs a second limb
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, q1_linear(x, bits, scale, 16))


@pytest.mark.parametrize("xmag,smag", [(7, 11), (20, 40), (30, 12), (45, 20), (62, 62)])
def test_q1_limb_envelopes_and_int64_scales(gpu, xmag, smag):
    N, nb = 48, 6
    seed = xmag * 100 + smag
    bits = prng.uniform_bytes(seed, 1, (N, nb, 16))
    scale = prng.uniform_int(seed, 2, (N, nb), -(1 << smag), 1 << smag)
    x = prng.uniform_int(seed, 3, (2, nb * 128), -(1 << xmag), 1 << xmag)
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, q1_linear(x, bits, scale, 16))


def test_q1_wrap_kat(gpu):
    x = np.zeros((1, 128), dtype=np.int64)
    x[0, 0] = 1 << 62
    bits = np.zeros((3, 1, 16), dtype=np.uint8)
    bits[:, 0, 0] = 1
    scale = np.array([[3], [-3], [4]], dtype=np.int64)
    assert list(gpu.q1_apply_gpu(x, bits, scale, 1)[0]) == [-(1 << 61), 1 << 61, 0]


@pytest.mark.parametrize("frac", [0, 1, 31, 62, 63, 64])
def test_q1_extrema_and_frac(gpu, frac):
    rng = np.random.default_rng(frac)
    N, nb = 20, 2
    bits = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    scale = rng.integers(I64_MIN, I64_MAX, size=(N, nb), dtype=np.int64)
    x = rng.integers(I64_MIN, I64_MAX, size=(2, nb * 128), dtype=np.int64)
    x[0, :4] = [I64_MIN, I64_MAX, 0, -1]
    got = gpu.q1_apply_gpu(x, bits, scale, frac)
    assert got is not None and np.array_equal(got, q1_linear_bigint(x, bits, scale, frac))


def test_q1_resident_equals_per_call_and_i32_registration(gpu):
    N, nb = 300, 12
    bits = prng.uniform_bytes(5, 1, (N, nb, 16))
    scale = prng.uniform_int(5, 2, (N, nb), -(1 << 20), 1 << 20)
    x = prng.uniform_int(5, 3, (1, nb * 128), -(1 << 18), 1 << 18)
    h64 = gpu.q1_register_weight(bits, scale)
    h32 = gpu.q1_register_weight(bits, scale.astype(np.int32))
    assert h64 is not None and h32 is not None
    want = q1_linear(x, bits, scale, 16)
    assert np.array_equal(gpu.q1_apply_resident(h64, x, N, nb, 16), want)
    assert np.array_equal(gpu.q1_apply_resident(h32, x, N, nb, 16), want)
    assert np.array_equal(gpu.q1_apply_gpu(x, bits, scale, 16), want)
    info = gpu.gpu_memory_info()
    assert info["resident_weight_bytes"] > 0
    gpu.q1_free_weights()
    assert gpu.gpu_memory_info()["resident_weight_bytes"] == 0


def test_q1_c1_shape_int8_activations(gpu):
    """Config 1: 4096x4096, x int8-range in int64, codec-range scales (round(fp16 * 2^16))."""
    N = K = 4096
    nb = K // 128
    bits = prng.uniform_bytes(11, 1, (N, nb, 16))
    h = prng.stream(11, 2, N * nb).astype(np.uint16) & np.uint16(0x7BFF)   # finite fp16 bit patterns
    sgn = np.where(prng.stream(11, 4, N * nb) & np.uint64(1), -1, 1)
    v = h.view(np.float16).astype(np.float64) * sgn
    scale = np.rint(v * 65536.0).astype(np.int64).reshape(N, nb)
    x = prng.uniform_int(11, 3, (1, K), -127, 128)
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, q1_linear(x, bits, scale, 16))


@pytest.mark.parametrize("nb,xmag,smag", [(12, 7, 20), (12, 40, 20), (8, 7, 40), (20, 40, 40)])
def test_q1_large_single_token_persistent_waves(gpu, nb, xmag, smag):
    """Single-token launches of more than 65536 tiles on one weight run persistent waves that walk tile groups
    gi, gi + W, ... with the slab pipeline running across group boundaries: a ragged last tile and group
    (N = 16 * 65539 + 3), odd and even slab counts (nb 12 -> 3 slabs, 20 -> 5, 8 -> 2), one-limb (|x| < 2^7) and
    multi-limb activations, int32 and int64 scales. Checked against the C restatement of the Q1 linear."""
    from oracle import c_oracle
    N = 16 * 65539 + 3
    rng = np.random.default_rng(nb * 100 + xmag + smag)
    bits = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    scale = rng.integers(-(1 << smag), 1 << smag, size=(N, nb), dtype=np.int64)
    x = rng.integers(-(1 << xmag) + 1, 1 << xmag, size=(1, nb * 128), dtype=np.int64)
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    want = c_oracle.q1_linear(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, want)
