"""Q1_0 GEMM path (T >= 8 tokens: int8 MFMA with tokens in the M dimension) vs the oracle, byte for byte."""
import numpy as np
import pytest

from oracle import c_oracle, prng
from oracle.q1 import q1_linear, q1_linear_bigint

pytestmark = pytest.mark.gpu
I64_MIN, I64_MAX = -(1 << 63), (1 << 63) - 1


@pytest.mark.parametrize("N,nb,T", [(16, 1, 8), (37, 3, 9), (200, 5, 64), (1000, 8, 100), (129, 32, 300),
                                    (4096, 32, 64)])
def test_gemm_shapes(gpu, N, nb, T):
    seed = N * 7 + nb * 3 + T
    bits = prng.uniform_bytes(seed, 1, (N, nb, 16))
    scale = prng.uniform_int(seed, 2, (N, nb), -(1 << 11), 1 << 11)
    x = prng.uniform_int(seed, 3, (T, nb * 128), -(1 << 20), 1 << 20)
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, c_oracle.q1_linear(x, bits, scale, 16))


@pytest.mark.parametrize("xmag,smag", [(7, 11), (23, 11), (24, 40), (30, 12), (45, 20), (62, 62)])
def test_gemm_limb_paths_and_int64_scales(gpu, xmag, smag):
    """int32 epilogue (<= 3 limbs) and the int64 one (more limbs / 64-bit scales)."""
    N, nb, T = 80, 6, 33
    seed = xmag * 100 + smag
    bits = prng.uniform_bytes(seed, 1, (N, nb, 16))
    scale = prng.uniform_int(seed, 2, (N, nb), -(1 << smag), 1 << smag)
    x = prng.uniform_int(seed, 3, (T, nb * 128), -(1 << xmag), 1 << xmag)
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, q1_linear(x, bits, scale, 16))


def test_gemm_mixed_token_magnitudes(gpu):
    """Tokens of one MFMA tile needing different limb counts (per-token limb masking)."""
    N, nb, T = 64, 4, 48
    bits = prng.uniform_bytes(21, 1, (N, nb, 16))
    scale = prng.uniform_int(21, 2, (N, nb), -(1 << 15), 1 << 15)
    x = prng.uniform_int(21, 3, (T, nb * 128), -(1 << 6), 1 << 6)
    big = prng.uniform_int(21, 4, (T, nb * 128), -(1 << 40), 1 << 40)
    x[::5] = big[::5]
    x[7, 130] = (1 << 62)
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, q1_linear(x, bits, scale, 16))


@pytest.mark.parametrize("frac", [0, 1, 31, 63, 64])
def test_gemm_extrema_and_frac(gpu, frac):
    rng = np.random.default_rng(100 + frac)
    N, nb, T = 24, 2, 16
    bits = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    scale = rng.integers(I64_MIN, I64_MAX, size=(N, nb), dtype=np.int64)
    x = rng.integers(I64_MIN, I64_MAX, size=(T, nb * 128), dtype=np.int64)
    x[0, :4] = [I64_MIN, I64_MAX, 0, -1]
    got = gpu.q1_apply_gpu(x, bits, scale, frac)
    assert got is not None and np.array_equal(got, q1_linear_bigint(x, bits, scale, frac))


def test_gemm_resident_matches_matvec_rows(gpu):
    """The same resident weight through the GEMM (T = 40) and the matvec (T = 1 per row) paths."""
    N, nb = 300, 12
    bits = prng.uniform_bytes(6, 1, (N, nb, 16))
    scale = prng.uniform_int(6, 2, (N, nb), -(1 << 20), 1 << 20)
    x = prng.uniform_int(6, 3, (40, nb * 128), -(1 << 18), 1 << 18)
    h = gpu.q1_register_weight(bits, scale)
    full = gpu.q1_apply_resident(h, x, N, nb, 16)
    rows = np.concatenate([gpu.q1_apply_resident(h, x[t:t + 1], N, nb, 16) for t in range(0, 40, 7)])
    assert np.array_equal(full[::7], rows)
    assert np.array_equal(full, q1_linear(x, bits, scale, 16))
    gpu.q1_free_weights()


def test_gemm_config3_shape(gpu):
    """Config 3 projection shape: M = 2048 tokens x 4096 -> 4096 (normed-activation magnitudes)."""
    N = K = 4096
    T = 2048
    bits = prng.uniform_bytes(31, 1, (N, K // 128, 16))
    scale = prng.uniform_int(31, 2, (N, K // 128), 1, 1 << 12)
    x = prng.uniform_int(31, 3, (T, K), -(1 << 19), 1 << 19)
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, c_oracle.q1_linear(x, bits, scale, 16))


@pytest.mark.parametrize("frac", [16, 24, 31])
def test_gemm_high_dword_epilogue_extremes(gpu, frac):
    """Scales at +-(2^(frac-1) - 1), the largest the high-dword epilogue takes, with activations at the 3-limb
    cap and all-one / all-zero bit rows: |S| ~ 2^30 per block, so the 32-bit partial is folded every 2 blocks."""
    cap3 = 127 * (1 + 256 + 65536)
    N, nb, T = 48, 32, 72
    rng = np.random.default_rng(frac)
    bits = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    bits[:8] = 0xFF
    bits[8:16] = 0
    smax = (1 << (frac - 1)) - 1
    scale = rng.choice(np.array([smax, -smax, smax - 1, 1], dtype=np.int64), size=(N, nb))
    scale[:4] = smax
    scale[8:12] = -smax
    x = rng.choice(np.array([cap3, -cap3, cap3 - 1, 0], dtype=np.int64), size=(T, nb * 128))
    x[:16] = cap3
    x[16:24] = -cap3
    got = gpu.q1_apply_gpu(x, bits, scale, frac)
    assert got is not None and np.array_equal(got, q1_linear(x, bits, scale, frac))


# ---- T >= 256: the +-1 sign-copy kernel (int32 scales under 2^(frac-1)) -----------------------------------------
@pytest.mark.parametrize("N,nb,T", [(129, 32, 300), (1000, 8, 256), (4096, 32, 512), (72, 3, 1000)])
def test_gemm_sign_copy_shapes(gpu, N, nb, T):
    seed = N * 11 + nb * 5 + T
    bits = prng.uniform_bytes(seed, 1, (N, nb, 16))
    scale = prng.uniform_int(seed, 2, (N, nb), -(1 << 11), 1 << 11)
    x = prng.uniform_int(seed, 3, (T, nb * 128), -(1 << 22), 1 << 22)
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, c_oracle.q1_linear(x, bits, scale, 16))


@pytest.mark.parametrize("frac", [16, 31])
def test_gemm_sign_copy_epilogue_extremes(gpu, frac):
    """As the high-dword extremes above, at T = 320: |S| ~ 2^30 per block, scales at +-(2^(frac-1) - 1)."""
    cap3 = 127 * (1 + 256 + 65536)
    N, nb, T = 48, 32, 320
    rng = np.random.default_rng(50 + frac)
    bits = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    bits[:8] = 0xFF
    bits[8:16] = 0
    smax = (1 << (frac - 1)) - 1
    scale = rng.choice(np.array([smax, -smax, smax - 1, 1], dtype=np.int64), size=(N, nb))
    scale[:4] = smax
    scale[8:12] = -smax
    x = rng.choice(np.array([cap3, -cap3, cap3 - 1, 0], dtype=np.int64), size=(T, nb * 128))
    x[:16] = cap3
    x[16:24] = -cap3
    got = gpu.q1_apply_gpu(x, bits, scale, frac)
    assert got is not None and np.array_equal(got, q1_linear(x, bits, scale, frac))


def test_gemm_sign_copy_with_wide_slabs(gpu):
    """Some slabs need more than 3 limbs on some token tiles: those blocks go to the wide kernel, which adds into
    the same outputs."""
    N, nb, T = 200, 16, 384
    bits = prng.uniform_bytes(77, 1, (N, nb, 16))
    scale = prng.uniform_int(77, 2, (N, nb), -(1 << 12), 1 << 12)
    x = prng.uniform_int(77, 3, (T, nb * 128), -(1 << 20), 1 << 20)
    big = prng.uniform_int(77, 4, (T, nb * 128), -(1 << 45), 1 << 45)
    x[100:140, 512:1024] = big[100:140, 512:1024]           # slab 1 of token tiles 1 and 2
    x[300, 1900] = (1 << 62)
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, q1_linear(x, bits, scale, 16))


def test_gemm_sign_copy_resident_lifecycle(gpu):
    """The sign copy is made once per resident weight on its first T >= 256 use (N * K bytes), reused, and
    released with the weight."""
    N, nb, T = 300, 12, 260
    bits = prng.uniform_bytes(8, 1, (N, nb, 16))
    scale = prng.uniform_int(8, 2, (N, nb), -(1 << 12), 1 << 12)
    x = prng.uniform_int(8, 3, (T, nb * 128), -(1 << 21), 1 << 21)
    gpu.q1_free_weights()
    h = gpu.q1_register_weight(bits, scale)
    base = gpu.gpu_memory_info()["resident_weight_bytes"]
    small = gpu.q1_apply_resident(h, x[:40], N, nb, 16)
    assert gpu.gpu_memory_info()["resident_weight_bytes"] == base
    want = q1_linear(x, bits, scale, 16)
    assert np.array_equal(small, want[:40])
    for _ in range(2):
        assert np.array_equal(gpu.q1_apply_resident(h, x, N, nb, 16), want)
        assert gpu.gpu_memory_info()["resident_weight_bytes"] == base + N * nb * 128
    gpu.q1_free_weights()
    assert gpu.gpu_memory_info()["resident_weight_bytes"] == 0


@pytest.mark.parametrize("nb,s", [(32, 4095), (32, 8191), (96, 1365), (96, 2730), (32, 16383)])
def test_gemm_sign_copy_partial_ranges(gpu, nb, s):
    """The multi-weight sign-copy kernel sums each block's floor into an int32 partial without folding, over all
    blocks or over each half (two partials); the host uses it only where the worst-case sum (|S| < 2^30 at 3 limbs
    times the row's sum of |scale| over the range) stays below 2^31. Uniform |scale| = s at the largest value
    that allows one partial and two partials (nb 32 and 96), and one that allows neither (the folded kernel runs);
    activations at the 3-limb maximum, rows of all-ones bits, mixed scale signs."""
    cap3 = 127 * (1 + 256 + 65536)
    N, T = 48, 320
    rng = np.random.default_rng(nb * 7 + s)
    bits = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    bits[:8] = 0xFF
    bits[8:12] = 0
    scale = np.full((N, nb), s, dtype=np.int64)
    scale[16:32] *= rng.choice(np.array([1, -1], dtype=np.int64), size=(16, nb))
    scale[40:] = -s
    x = rng.choice(np.array([cap3, -cap3, cap3 - 1, 0], dtype=np.int64), size=(T, nb * 128))
    x[:16] = cap3
    x[16:24] = -cap3
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, q1_linear(x, bits, scale, 16))


# ---- 8 <= T <= 64: the batched-decode kernel (one token tile, K ranges of 1 / 2 / 4 blocks) ----------------------
@pytest.mark.parametrize("N,nb,T", [(300, 12, 8), (300, 12, 16), (257, 5, 17), (1000, 8, 32), (64, 13, 33),
                                    (513, 4, 48), (4096, 32, 64), (40, 96, 31)])
def test_gemm_batched_decode_shapes(gpu, N, nb, T):
    seed = N * 13 + nb * 7 + T
    bits = prng.uniform_bytes(seed, 1, (N, nb, 16))
    scale = prng.uniform_int(seed, 2, (N, nb), -(1 << 13), 1 << 13)
    x = prng.uniform_int(seed, 3, (T, nb * 128), -(1 << 22), 1 << 22)
    x[T // 2, :] = 0                                  # a token whose slabs need no limbs
    got = gpu.q1_apply_gpu(x, bits, scale, 16)
    assert got is not None and np.array_equal(got, c_oracle.q1_linear(x, bits, scale, 16))


@pytest.mark.parametrize("frac,T", [(16, 32), (31, 20), (24, 64)])
def test_gemm_batched_decode_epilogue_extremes(gpu, frac, T):
    """Scales at +-(2^(frac-1) - 1) and activations at the 3-limb cap: |q| ~ 2^29 per block, so the host takes
    ranges of at most 2 blocks for the int32 partial; one slab needing 4 limbs goes through the wide path."""
    cap3 = 127 * (1 + 256 + 65536)
    N, nb = 96, 16
    rng = np.random.default_rng(frac + T)
    bits = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    bits[:8] = 0xFF
    bits[8:16] = 0
    smax = (1 << (frac - 1)) - 1
    scale = rng.choice(np.array([smax, -smax, smax - 1, 1], dtype=np.int64), size=(N, nb))
    x = rng.choice(np.array([cap3, -cap3, cap3 - 1, 0], dtype=np.int64), size=(T, nb * 128))
    x[:4] = cap3
    x[4:8] = -cap3
    x[T - 1, 5 * 128 + 3] = cap3 + 1                  # slab 1 needs 4 limbs for every token of the tile
    got = gpu.q1_apply_gpu(x, bits, scale, frac)
    assert got is not None and np.array_equal(got, q1_linear(x, bits, scale, frac))
