"""Pin the Q4_K / Q6_K oracle (CPU only)."""
import ctypes
from pathlib import Path

import numpy as np
import pytest

from oracle import c_oracle, qk

REF = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libnmc_qk_kernel.so"


def test_fp16_fixed_matches_python_round_for_every_finite_fp16():
    h = np.arange(0, 1 << 16, dtype=np.int64)
    e = (h >> 10) & 31
    h = h[e != 31]
    for fw in (16, 24):
        got = qk.fp16_fixed(h[::7], fw)
        want = [int(round(float(v) * (1 << fw))) for v in h[::7].astype(np.uint16).view(np.float16)]
        assert list(got) == want
        assert [c_oracle.fp16_fixed(int(x), fw) for x in h[::97]] == [int(round(float(v) * (1 << fw))) for v in
                                                                      h[::97].astype(np.uint16).view(np.float16)]


def test_q4k_hand_built_block_closed_form():
    # d = 1.0 (0x3C00), dmin = 0.5 (0x3800); sub-block j scale j+1, min j; quants = position % 16
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:4] = [0x00, 0x38]
    sc = np.array([j + 1 for j in range(8)])
    mn = np.arange(8)
    s = np.zeros(12, dtype=np.int64)
    for j in range(4):
        s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    blk[4:16] = s.astype(np.uint8)
    q = np.arange(256) % 16
    qs = np.zeros(128, dtype=np.int64)
    for g in range(4):
        qs[32 * g:32 * g + 32] = q[64 * g:64 * g + 32] | (q[64 * g + 32:64 * g + 64] << 4)
    blk[16:] = qs.astype(np.uint8)
    w = qk.dequant(blk, 1, 1, 0, 16)[0]
    want = [(1 << 16) * (i // 32 + 1) * (i % 16) - (1 << 15) * (i // 32) for i in range(256)]
    assert list(w) == want


@pytest.mark.parametrize("qtype", [0, 1])
def test_numpy_linear_equals_compiled_reference_kernel(qtype):
    if not REF.exists():
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    so = ctypes.CDLL(str(REF))
    f = so.qk_linear
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                  ctypes.c_int, ctypes.c_void_p]
    out_f, nb, T = 7, 3, 4
    raw = qk.random_blocks(5, 10 + qtype, out_f, nb, qtype)
    x = np.random.default_rng(qtype).integers(-(1 << 30), 1 << 30, size=(T, nb * 256), dtype=np.int64)
    out = np.empty((T, out_f), dtype=np.int64)
    f(raw.ctypes.data, x.ctypes.data, T, out_f, nb, 24, qtype, out.ctypes.data)
    W = qk.dequant(raw, out_f, nb, qtype, 24)
    assert np.array_equal(out, qk.linear(x, W, 24))
    assert np.array_equal(c_oracle.qk_linear(raw, x, out_f, nb, 24, qtype), out)


def test_negative_floor_division():
    # north-mini-code/tests/test_qk_native.py:38-44 style: results below zero floor toward -inf
    raw = qk.random_blocks(9, 1, 3, 1, 0)
    x = -np.ones((1, 256), dtype=np.int64)
    W = qk.dequant(raw, 3, 1, 0, 24)
    assert list(qk.linear(x, W, 24)[0]) == [int(v) >> 24 for v in -W.astype(object).sum(axis=1)]


def test_topk_lowest_index_on_ties():
    assert list(qk.topk_lowidx(np.array([5, 7, 7, 1, 7]), 2)) == [1, 2]


def test_moe_grouped_equals_per_token_and_c_linear():
    E, k, d, e_ffn, T = 6, 2, 256, 256, 5
    raws = {e: dict(gate=qk.random_blocks(1, 100 + 3 * e, e_ffn, 1, 0), up=qk.random_blocks(1, 101 + 3 * e, e_ffn, 1, 0),
                    down=qk.random_blocks(1, 102 + 3 * e, d, 1, 1)) for e in range(E)}
    deq = {e: dict(gate=qk.dequant(r["gate"], e_ffn, 1, 0, 24), up=qk.dequant(r["up"], e_ffn, 1, 0, 24),
                   down=qk.dequant(r["down"], d, 1, 1, 24)) for e, r in raws.items()}
    h = np.random.default_rng(0).integers(-(1 << 16), 1 << 16, size=(T, d), dtype=np.int64)
    logits = np.random.default_rng(1).integers(-(1 << 20), 1 << 20, size=(T, E), dtype=np.int64)
    sel, gates = qk.moe_route(logits, k, 16)
    ref = qk.moe_ffn(h, sel, gates, deq, 16, 24)
    assert np.array_equal(qk.moe_ffn_grouped(h, sel, gates, deq, 16, 24, qk.linear), ref)
    shapes = {"gate": (e_ffn, 1, 0), "up": (e_ffn, 1, 0), "down": (d, 1, 1)}
    rawc = {e: {n: (r[n], *shapes[n]) for n in r} for e, r in raws.items()}
    lin = lambda x, w, fw: c_oracle.qk_linear(w[0], x, w[1], w[2], fw, w[3])
    assert np.array_equal(qk.moe_ffn_grouped(h, sel, gates, rawc, 16, 24, lin), ref)


def test_moe_composition_tracks_float_math():
    """The integer MoE equals the real-valued formula sum_j g_j * down(silu(gate h) * up h) within fixed-point
    rounding (the reference gates its MoE the same way: int vs float, north-mini-code/tests/test_cohere2_moe.py:
    44-51, rel < 5e-3). A dropped term, a sign error or a transposed weight fails by orders of magnitude."""
    E, k, d, e_ffn, T, fa, fw = 5, 2, 256, 256, 4, 16, 24
    raws = {e: dict(gate=qk.random_blocks(2, 200 + 3 * e, e_ffn, 1, 0), up=qk.random_blocks(2, 201 + 3 * e, e_ffn, 1, 0),
                    down=qk.random_blocks(2, 202 + 3 * e, d, 1, 1)) for e in range(E)}
    deq = {e: {n: qk.dequant(r[n], e_ffn if n != "down" else d, 1, 0 if n != "down" else 1, fw) for n in r}
           for e, r in raws.items()}
    rng = np.random.default_rng(3)
    h = rng.integers(-(1 << 19), 1 << 19, size=(T, d), dtype=np.int64)
    logits = rng.integers(-(1 << 17), 1 << 17, size=(T, E), dtype=np.int64)
    sel, gates = qk.moe_route(logits, k, fa)
    got = qk.moe_ffn(h, sel, gates, deq, fa, fw).astype(np.float64) / 2.0 ** fa
    hf = h.astype(np.float64) / 2.0 ** fa
    want = np.zeros((T, d))
    for t in range(T):
        for j, e in enumerate(sel[t]):
            W = {n: deq[int(e)][n].astype(np.float64) / 2.0 ** fw for n in ("gate", "up", "down")}
            g, u = W["gate"] @ hf[t], W["up"] @ hf[t]
            a = g / (1.0 + np.exp(-g)) * u
            gate = 1.0 / (1.0 + np.exp(-logits[t, e] / 2.0 ** fa))
            want[t] += gate * (W["down"] @ a)
    rel = np.max(np.abs(got - want)) / np.max(np.abs(want))
    assert rel < 5e-3, rel


def test_interleaved_rope_is_neox_on_a_permuted_head():
    """Pairwise (2i, 2i+1) rotation == the NeoX (i, i + hd/2) rotation after the even/odd -> halves permutation."""
    from oracle.rope import apply_interleaved, apply_neox, build_rope_tables
    rng = np.random.default_rng(12)
    hd, seq = 16, 5
    cos, sin = build_rope_tables(seq, hd, base=50000, frac=16)
    x = rng.integers(-(1 << 30), 1 << 30, size=(3, seq, hd), dtype=np.int64)
    perm = np.concatenate([np.arange(0, hd, 2), np.arange(1, hd, 2)])
    got = apply_interleaved(x, cos, sin, 16)
    want = np.empty_like(x)
    want[..., perm] = apply_neox(x[..., perm], cos, sin, 16)
    assert np.array_equal(got, want)


def test_router_logits_guard():
    from oracle.nmc_block import router_logits
    h = np.array([[1 << 40, 1 << 40]], dtype=np.int64)
    assert router_logits(h, np.array([[3, -2]], dtype=np.int64), 4).tolist() == [[(1 << 40) >> 4]]
    with pytest.raises(OverflowError):
        router_logits(h, np.array([[1 << 30, 1 << 30]], dtype=np.int64), 4)
