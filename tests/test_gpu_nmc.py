"""north-mini-code Q4_K / Q6_K linear and the ragged MoE block on gfx950 vs the oracle (after
north-mini-code/tests/test_qk_cuda.py:28-37, :52-56, :535-587, :648-685)."""
import numpy as np
import pytest

from oracle import c_oracle, prng, qk

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qkg():
    from integer_inference_engine_amd import qk_gpu
    assert qk_gpu.available()
    return qk_gpu


@pytest.mark.parametrize("qtype,out_f,nb,T,xmag", [(0, 33, 2, 1, 16), (1, 70, 3, 5, 16), (0, 128, 8, 17, 30),
                                                   (1, 64, 1, 3, 55), (0, 5, 1, 2, 62),
                                                   # int8-MFMA path: token tiles of 16 with ragged tails, 1..5
                                                   # limbs, and 2^39 (beyond 5 limbs: the VALU kernel takes over)
                                                   (0, 96, 4, 40, 30), (1, 80, 2, 33, 36), (0, 16, 1, 16, 38),
                                                   (1, 48, 2, 7, 39), (0, 200, 3, 1, 6), (1, 130, 1, 18, 20)])
def test_qk_linear_matches_oracle(qkg, qtype, out_f, nb, T, xmag):
    raw = qk.random_blocks(out_f, qtype, out_f, nb, qtype)
    x = prng.uniform_int(xmag, T, (T, nb * 256), -(1 << xmag), 1 << xmag)
    W = qk.dequant(raw, out_f, nb, qtype, 24)
    try:
        want = qk.linear(x, W, 24)
    except OverflowError:
        assert qkg.qk_linear(raw, x, out_f, nb, 24, qtype) is None
        return
    assert np.array_equal(qkg.qk_linear(raw, x, out_f, nb, 24, qtype), want)


def test_resident_grouped_equals_individual(qkg):
    raws = [qk.random_blocks(3, 20 + i, n, 4, i % 2) for i, n in enumerate((48, 16, 16))]
    hs = [qkg.register_weight(r, n, 4, i % 2) for i, (r, n) in enumerate(zip(raws, (48, 16, 16)))]
    x = prng.uniform_int(3, 30, (3, 1024), -(1 << 16), 1 << 16)
    outs = qkg.apply_resident_grouped(hs, x, (48, 16, 16), 24, phase_ids=(1, 2, 3))
    for i, (h, r, n) in enumerate(zip(hs, raws, (48, 16, 16))):
        want = qk.linear(x, qk.dequant(r, n, 4, i % 2, 24), 24)
        assert np.array_equal(outs[i], want)
        assert np.array_equal(qkg.apply_resident(h, x, n, 24), want)
        assert np.array_equal(qkg.apply_resident_dp4a(h, x, n, 24, i % 2), want)
    qkg.free_all()
    assert qkg.resident_count() == 0


def _experts(seed, E, d, e_ffn, dq=(0.002, 0.01, 0.005)):
    kw = dict(dlo=dq[0], dhi=dq[1], dminhi=dq[2])
    return [dict(gate=qk.random_blocks(seed, 100 + 3 * e, e_ffn, d // 256, 0, **kw),
                 up=qk.random_blocks(seed, 101 + 3 * e, e_ffn, d // 256, 0, **kw),
                 down=qk.random_blocks(seed, 102 + 3 * e, d, e_ffn // 256, 1, **kw)) for e in range(E)]


def _run_moe(qkg, seed, E, k, d, e_ffn, T, *, fast_oracle=False, hmag=16, oracle=True, dq=(0.002, 0.01, 0.005)):
    ex = _experts(seed, E, d, e_ffn, dq)
    hs = [dict(gate=qkg.register_weight(x["gate"], e_ffn, d // 256, 0),
               up=qkg.register_weight(x["up"], e_ffn, d // 256, 0),
               down=qkg.register_weight(x["down"], d, e_ffn // 256, 1)) for x in ex]
    h = prng.uniform_int(seed, 7, (T, d), -(1 << hmag), 1 << hmag)
    logits = prng.uniform_int(seed, 8, (T, E), -(1 << 20), 1 << 20)
    sel, gates = qk.moe_route(logits, k, 16)
    flat = sel.reshape(-1)
    got = qkg.moe_ffn_batched([hs[e]["gate"] for e in flat], [hs[e]["up"] for e in flat],
                              [hs[e]["down"] for e in flat], T, k, h, gates, d, e_ffn, 16, 24)
    used = sorted(set(int(e) for e in flat))
    if not oracle:
        qkg.free_all()
        return got, None
    if fast_oracle:
        raw = {e: dict(gate=(ex[e]["gate"], e_ffn, d // 256, 0), up=(ex[e]["up"], e_ffn, d // 256, 0),
                       down=(ex[e]["down"], d, e_ffn // 256, 1)) for e in used}
        lin = lambda x, w, fw: c_oracle.qk_linear(w[0], x, w[1], w[2], fw, w[3])
        want = qk.moe_ffn_grouped(h, sel, gates, raw, 16, 24, lin)
    else:
        deq = {e: dict(gate=qk.dequant(ex[e]["gate"], e_ffn, d // 256, 0, 24),
                       up=qk.dequant(ex[e]["up"], e_ffn, d // 256, 0, 24),
                       down=qk.dequant(ex[e]["down"], d, e_ffn // 256, 1, 24)) for e in used}
        want = qk.moe_ffn(h, sel, gates, deq, 16, 24)
    qkg.free_all()
    return got, want


def test_moe_batched_small_matches_oracle(qkg):
    got, want = _run_moe(qkg, 1, E=8, k=3, d=512, e_ffn=256, T=5)
    assert got is not None and np.array_equal(got, want)


@pytest.mark.parametrize("hmag,T,E,dq", [(16, 23, 4, (0.002, 0.01, 0.005)), (33, 9, 3, (1e-4, 1e-4, 5e-5)),
                                         (41, 6, 4, (6e-8, 6e-8, 6e-8)), (2, 17, 2, (0.002, 0.01, 0.005)),
                                         (45, 5, 3, (0.002, 0.01, 0.005))])
def test_moe_fused_expert_kernels_limb_and_token_groups(qkg, hmag, T, E, dq):
    """The fused expert kernels over every branch: more than 4 tokens per expert (several token groups), five
    limbs (2^33: the second MFMA row group), activations beyond five limbs (2^41: the exact VALU fallback,
    selected on the device; tiny block scales keep the oracle's int64 results in range), one-limb activations,
    and a case whose results leave int64 (2^45 with ordinary scales: refused as the oracle raises)."""
    try:
        got, want = _run_moe(qkg, hmag + T, E=E, k=2, d=512, e_ffn=256, T=T, hmag=hmag, dq=dq)
    except OverflowError:                                             # the oracle raises: the producer must refuse
        qkg.free_all()
        got, _ = _run_moe(qkg, hmag + T, E=E, k=2, d=512, e_ffn=256, T=T, hmag=hmag, oracle=False, dq=dq)
        assert got is None
        return
    assert got is not None and np.array_equal(got, want)


def test_moe_single_token_equals_batched_row(qkg):
    ex = _experts(2, 4, 256, 256)
    hs = [dict(gate=qkg.register_weight(x["gate"], 256, 1, 0), up=qkg.register_weight(x["up"], 256, 1, 0),
               down=qkg.register_weight(x["down"], 256, 1, 1)) for x in ex]
    h = prng.uniform_int(2, 7, (2, 256), -(1 << 16), 1 << 16)
    sel = np.array([[0, 2], [3, 0]])
    gates = np.array([[30000, 5000], [60000, 100]], dtype=np.int64)
    flat = sel.reshape(-1)
    b = qkg.moe_ffn_batched([hs[e]["gate"] for e in flat], [hs[e]["up"] for e in flat], [hs[e]["down"] for e in flat],
                            2, 2, h, gates, 256, 256, 16, 24)
    for t in range(2):
        one = qkg.moe_ffn([hs[e]["gate"] for e in sel[t]], [hs[e]["up"] for e in sel[t]],
                          [hs[e]["down"] for e in sel[t]], h[t], gates[t], 256, 256, 16, 24)
        assert np.array_equal(one, b[t])
    qkg.free_all()


def test_config4_moe_block_byte_exact(qkg):
    """Config 4: hidden 2048, 128 experts, top-8, expert FFN 768, Q4_K gate/up + Q6_K down, 64 tokens with
    seeded integer router logits (ragged per-expert groups). Oracle: the exact composition evaluated expert by
    expert with the C int128 linear (pinned to the big-int form in tests/test_oracle_qk.py)."""
    got, want = _run_moe(qkg, 4, E=128, k=8, d=2048, e_ffn=768, T=64, fast_oracle=True)
    assert got is not None
    bad = np.count_nonzero(got != want)
    assert bad == 0, f"{bad} mismatches"


@pytest.mark.parametrize("fw", [0, 1, 7, 16, 24, 29, 40, 41, 45])
def test_fp16_fixed_device_form_is_exhaustively_exact(fw):
    """The kernels' fp16 -> fixed conversion (double-precision form, integer rule for exponent 31 and fw > 40)
    against the oracle's integer rule over all 65536 fp16 bit patterns (nmc_qk_kernel.c:16-39)."""
    import ctypes
    from integer_inference_engine_amd import _lib
    so = _lib.lib()
    h = np.arange(1 << 16, dtype=np.uint16)
    got = np.empty(1 << 16, dtype=np.int64)
    assert so.imie_fp16_fixed_probe(h.ctypes.data, h.size, fw, got.ctypes.data) == 0
    want = qk.fp16_fixed(h, fw)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"fw={fw}: {bad.size} mismatches, first h={int(h[bad[0]]):#06x} got {got[bad[0]]} want {want[bad[0]]}"
