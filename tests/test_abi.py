"""The C-ABI library loads, exports every declared symbol, and its host-side repack is correct (CPU only)."""
import ctypes
import re
from pathlib import Path

import numpy as np

from integer_inference_engine_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        for m in re.finditer(r"^\s*(?:[A-Za-z_][\w\s\*]*?)\b((?:bonsai|qk|imie)_\w+)\s*\(", h.read_text(), re.M):
            names.add(m.group(1))
    return names


def test_library_loads_and_exports_declared_symbols():
    so = _lib.lib()
    declared = _declared_symbols()
    assert declared, "no declarations found in include/*.h"
    missing = [n for n in sorted(declared) if not hasattr(so, n)]
    assert not missing, f"symbols declared in include/*.h but not exported: {missing}"
    assert set(_lib.SIGNATURES) <= declared, sorted(set(_lib.SIGNATURES) - declared)


def test_q1_repack_host_layout():
    so = _lib.lib()
    rng = np.random.default_rng(0)
    N, nb = 37, 6                      # ragged: pads rows to 48 and blocks to 8
    bits = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    scale = rng.integers(-(1 << 30), 1 << 30, size=(N, nb), dtype=np.int64)
    ntiles, nslabs = 3, 2
    bt = np.zeros((ntiles, nslabs, 64, 16), dtype=np.uint8)
    st = np.zeros((ntiles, nslabs, 64), dtype=np.int32)
    rc = so.imie_q1_repack_host(bits.ctypes.data, scale.ctypes.data, N, nb, 0, bt.ctypes.data, st.ctypes.data)
    assert rc == 0
    for tile in range(ntiles):
        for sl in range(nslabs):
            for lane in range(64):
                row, blk = tile * 16 + (lane & 15), sl * 4 + (lane >> 4)
                if row < N and blk < nb:
                    assert np.array_equal(bt[tile, sl, lane], bits[row, blk])
                    assert st[tile, sl, lane] == scale[row, blk]
                else:
                    assert not bt[tile, sl, lane].any() and st[tile, sl, lane] == 0


def test_exact_norm_helpers_host():
    """isqrt / reciprocal / 128-by-32 division used by the RMSNorm kernels, against Python big integers on
    random magnitudes and the edges (perfect squares and their neighbours, 2^64 - 1, power-of-two divisors)."""
    import math
    so = _lib.lib()
    rng = np.random.default_rng(7)
    vals = [0, 1, 2, 3, 4, (1 << 64) - 1, 1 << 64, (1 << 100) - 1, 1 << 100, (1 << 128) - 1]
    for r in [1, 2, 3, 1 << 20, (1 << 32) + 1, (1 << 50) - 3, (1 << 64) - 1]:
        vals += [r * r - 1, r * r, r * r + 1]
    for bits in range(1, 129, 3):
        vals += [int(rng.integers(0, 1 << 62)) << (bits - 62) if bits > 62 else int(rng.integers(0, 1 << bits))
                 for _ in range(6)]
    for v in vals:
        v &= (1 << 128) - 1
        assert so.imie_fx_isqrt_u128(v >> 64, v & ((1 << 64) - 1)) == math.isqrt(v), v
    for d in [1, 2, 3, 5, 7, 255, 4096, 12345, (1 << 32) - 1, 1 << 40, (1 << 63) + 11, (1 << 64) - 1] + \
             [int(x) for x in rng.integers(1, 1 << 62, size=200)]:
        assert so.imie_fx_recip_u64(d) == ((1 << 64) - 1) // d, d
    for d in [1, 3, 128, 4096, 4095, 12288, (1 << 32) - 1]:
        for v in vals[:40]:
            v &= (1 << 128) - 1
            assert so.imie_fx_div_u128(v >> 64, v & ((1 << 64) - 1), d) == (v // d) & ((1 << 64) - 1), (v, d)


def test_prologue_short_paths_host():
    """The double-precision short paths of the single-token matvec prologue against exact integer arithmetic: the
    isqrt below 2^52 (perfect squares and their neighbours up to the bound), n = floor((x << f) / rms) with the
    oracle's floor toward -inf (exact multiples, remainders of rms - 1, the edges of the bounds), and the
    one-exponential SiLU * up against the two-exponential form and the numpy oracle (fixedpoint.py:89-117)."""
    import math
    from oracle import fixedpoint as fx
    so = _lib.lib()
    rng = np.random.default_rng(11)
    vals = [0, 1, 2, 3, (1 << 52) - 1, (1 << 52), (1 << 60) + 5, (1 << 100) + 3]
    for r in [1, 2, 3, 1 << 13, (1 << 26) - 1, 1 << 26, 67108863, 94906265]:
        vals += [r * r - 1, r * r, r * r + 1]
    vals += [int(v) for v in rng.integers(0, 1 << 52, size=400)]
    for v in vals:
        if v >= 0:
            assert so.imie_fx_isqrt_fast(v >> 64, v & ((1 << 64) - 1)) == math.isqrt(v), v
    out = ctypes.c_int64()
    cases = []
    for frac in (1, 8, 16, 29):
        lim = 1 << (53 - frac)
        for rms in [1, 2, 3, 7, 65535, 65536, 1 << 26, (1 << 33) + 1, (1 << 51) - 1, 1 << 51]:
            xs = [0, 1, -1, lim - 1, -(lim - 1), lim, -lim, rms, -rms, 2 * rms - 1, -(2 * rms - 1)]
            xs += [int(v) for v in rng.integers(-lim, lim, size=60)]
            cases += [(x, frac, rms) for x in xs]
    fast = 0
    for x, frac, rms in cases:
        rc = so.imie_fx_norm_f64(x, frac, rms, ctypes.byref(out))
        inside = abs(x) < (1 << (53 - frac)) and rms < (1 << 51)
        assert rc == (1 if inside else 0), (x, frac, rms)
        if rc == 1:
            fast += 1
            assert out.value == (x << frac) // rms, (x, frac, rms)
    assert fast > 1000
    for frac in (8, 16, 24, 29):
        g = np.concatenate([rng.integers(-(1 << 40), 1 << 40, size=300), rng.integers(-(1 << 20), 1 << 20, size=300),
                            np.array([0, 1, -1, (1 << 63) - 1, -(1 << 63), -(1 << 63) + 1, 1 << frac, -(1 << frac)])])
        u = rng.integers(-(1 << 30), 1 << 30, size=g.size)
        want = fx.mulshift_wrap(fx.silu_wrap(g.astype(np.int64), frac), u.astype(np.int64), frac)
        for gi, ui, wi in zip(g.tolist(), u.tolist(), want.tolist()):
            assert so.imie_silu_mul_host(gi, ui, frac, 1) == wi, (gi, ui, frac)
            assert so.imie_silu_mul_host(gi, ui, frac, 0) == wi, (gi, ui, frac)


def test_softmax_short_paths_host():
    """The prefill softmax's short paths against the numpy oracle (fixedpoint.py:49-87): the exponential of a clipped
    difference d in [0, dclip] by one 32 x 32 product and the 32-bit cubic (both forms, every fraction width the
    kernels accept; the integer-part boundaries k * 2^frac and the clip edge included), and p = floor((e << frac)
    / Z) by the double quotient with exact correction (exact multiples, remainders of Z - 1, e at 0 and 2^frac,
    Z from 1 up to 2^52)."""
    from oracle import fixedpoint as fx
    so = _lib.lib()
    rng = np.random.default_rng(12)
    for frac in (1, 2, 8, 16, 24, 29):
        log2e, dclip = fx.scaled_log2e(frac), fx.d_clip(frac)
        ds = [0, 1, 2, dclip - 1, dclip] + [int(v) for v in rng.integers(0, dclip + 1, size=600)]
        ds += [max(0, min(dclip, ((k << frac) * (1 << frac)) // log2e + o)) for k in range(0, 40) for o in (-1, 0, 1)]
        want = fx.exp2_neg_fixed(np.array([(x * log2e) >> frac for x in ds], dtype=np.int64), frac)
        for x, w in zip(ds, want.tolist()):
            assert so.imie_exp_clipped_host(x, frac, 1) == w, (x, frac)
            assert so.imie_exp_clipped_host(x, frac, 0) == w, (x, frac)
        for z in [1, 2, 3, 1 << frac, (1 << frac) + 1, 12345677, (1 << 40) + 7, (1 << 52) - 1, 1 << 52]:
            es = [0, 1, (1 << frac) - 1, 1 << frac, z % (1 << frac)] + [int(v) for v in rng.integers(0, (1 << frac) + 1, size=60)]
            for e in es:
                assert so.imie_prob_div_host(e, frac, z) == (e << frac) // z, (e, frac, z)


def test_exports_every_symbol_the_reference_nmc_loader_requires():
    """north-mini-code/src/nmc/qk_cuda.py:39-72 (_REQUIRED_CUDA_SYMBOLS) and the ABI version it checks (:22, 83-92):
    the reference bridge binds this library unchanged."""
    names = """qk_cuda_abi_version qk_linear_cuda qk_cuda_available qk_register_weight qk_register_i64
    qk_resident_reserve qk_apply_resident qk_apply_resident_grouped qk_rmsnorm_router qk_attention_bank_create
    qk_attention_bank_import qk_attention_bank_apply qk_attention_bank_moe_configure qk_attention_bank_moe_bind
    qk_attention_bank_moe_begin qk_attention_bank_moe_continue qk_attention_bank_moe_export
    qk_attention_bank_workspace_bytes qk_attention_bank_reset qk_attention_bank_destroy qk_free_all
    qk_resident_count qk_resident_capacity qk_moe_workspace_allocations qk_moe_workspace_bytes
    qk_moe_workspace_release qk_moe_ffn qk_moe_ffn_batched qk_moe_ffn_batched_dp4a qk_profile_reset
    qk_profile_set_enabled qk_profile_snapshot""".split()
    assert len(names) == 32
    so = _lib.lib()
    assert [n for n in names if not hasattr(so, n)] == []
    assert so.qk_cuda_abi_version() == 5


def test_exports_every_symbol_the_reference_bonsai_loader_binds():
    """Every bonsai_* name bonsai/src/trinote/infer_int/gpu_native.py binds (:44-172, including the optional
    dp4a :55-64 and layout registrations :80-105), plus the ABI queries of bonsai_q1_gpu.cu:1970-1980: the
    reference loader pointed at this library finds all of them, so none of its optional paths falls back."""
    names = """bonsai_q1_linear_gpu bonsai_q1_linear_dp4a_gpu bonsai_q1_register_weight bonsai_q1_apply_resident
    bonsai_q1_free_weights bonsai_q1_register_weight_i32 bonsai_q1_register_weight_i32_gpu_layout
    bonsai_q1_register_weight_i32_bmma bonsai_gpu_mem_info bonsai_q1_resident_weight_bytes
    bonsai_gpu_reservation_create bonsai_gpu_reservation_free bonsai_rmsnorm_gpu bonsai_attention_prefill_gpu
    bonsai_buf_upload_i64 bonsai_prefill_forward_gpu bonsai_gpu_available bonsai_attention_decode_batched_gpu
    bonsai_decode_ctx_create bonsai_decode_ctx_seed_seq bonsai_decode_step bonsai_decode_ctx_free
    bonsai_gpu_abi_version bonsai_gpu_last_error_code bonsai_gpu_last_error""".split()
    so = _lib.lib()
    assert [n for n in names if not hasattr(so, n)] == []
    assert so.bonsai_gpu_abi_version() == 3


def test_dp4a_refusals_before_any_device_work():
    """bonsai_q1_linear_dp4a_gpu argument refusals (bonsai_q1_gpu.cu:2249: rc 1 for |L| outside 1..8 or empty
    shapes) are decided before the device is touched."""
    so = _lib.lib()
    x = np.zeros((1, 128), dtype=np.int64)
    bits = np.zeros((1, 1, 16), dtype=np.uint8)
    sc = np.ones((1, 1), dtype=np.int64)
    out = np.zeros((1, 1), dtype=np.int64)
    for L in (0, 9, -9):
        assert so.bonsai_q1_linear_dp4a_gpu(x.ctypes.data, bits.ctypes.data, sc.ctypes.data, 1, 1, 1, 16, L,
                                            out.ctypes.data) == 1
    assert so.bonsai_q1_linear_dp4a_gpu(x.ctypes.data, bits.ctypes.data, sc.ctypes.data, 0, 1, 1, 16, 4,
                                        out.ctypes.data) == 1
    assert so.bonsai_q1_register_weight_i32_bmma(bits.ctypes.data, sc.astype(np.int32).ctypes.data, 1, 1) == -1


def test_profile_metric_names_match_the_native_enum():
    """qk_profile_snapshot writes the counters in the order of the PM_* enum of csrc/nmc.hip; the Python names must
    match it one for one (qk_cuda.py:24-34 order)."""
    import re
    from pathlib import Path
    from integer_inference_engine_amd import qk_gpu
    src = (Path(__file__).resolve().parents[1] / "integer_inference_engine_amd/csrc/nmc.hip").read_text()
    body = re.search(r"enum \{ (PM_REG_CALLS.*?)PM_COUNT \};", src, re.S).group(1)
    native = [n.strip() for n in body.replace("\n", " ").split(",") if n.strip()]
    assert len(native) == len(qk_gpu.PROFILE_METRICS) == 28
    short = {"registration": "REG", "allocation": "ALLOC", "resident_apply": "RESIDENT", "grouped_apply": "GROUPED",
             "q_projection": "Q", "k_projection": "K", "v_projection": "V", "o_projection": "O",
             "other_projection": "OTHER"}
    for name, enum in zip(qk_gpu.PROFILE_METRICS, native):
        stem, _, unit = name.rpartition("_")
        assert enum == f"PM_{short.get(stem, stem.upper())}_{unit.upper()}", (name, enum)
