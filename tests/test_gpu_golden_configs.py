"""The five BASELINE configurations at their stated sizes on gfx950, against the oracle's committed digests
(tests/golden/configs.json, written by tests/golden/make_config_golden.py from the CPU oracle; the CPU suite
re-derives C1-C4 from the oracle in tests/test_golden_configs.py).

* C1: 4096x4096 Q1_0 matvec, codec-range int64 scales, int8-range x (reference_bonsai.py:149-219).
* C2: 8B-shape layer decode at position 4096 over a seeded kv8 cache: output and new K/V rows.
* C3: 8B-shape layer prefill over 2048 tokens (the sign-copy GEMMs and the causal kv8 attention at full length):
  output and all 2048 K/V rows (reference_bonsai.py:968-1065).
* C4: the MoE block, 64 tokens x top-8 of 128 experts (cohere2.py:162-188).
* C5: 36 layers, 32 sequences with contexts U[512, 32768] in the paged kv8 cache, 64 greedy steps: every token of
  the graph-replayed run, and per step the digest of all 32 logits rows (an eager step-by-step rerun, which also
  shows graph == eager) (reference_bonsai.py:1175-1310)."""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import configs as C
from tests.bonsai_gpu_harness import register_model

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "configs.json").read_text())


def _net(gpu, model, B, cap, with_head=False, n_layers=1):
    from integer_inference_engine_amd.resident import ResidentNet
    w, g = register_model(gpu, model, with_head=with_head)
    return ResidentNet(B=B, n_layers=n_layers, H=C.H, Hkv=C.HKV, hd=C.HD, d=C.D, dff=C.DFF, cap=cap, w=w, g=g,
                       page=64, kv32=True)


def test_c1_matvec_golden(gpu):
    x, bits, scale = C.c1_inputs()
    assert C.sha(gpu.q1_apply_gpu(x, bits, scale, 16)) == GOLDEN["c1"]["out_sha256"]
    h = gpu.q1_register_weight(bits, scale)
    assert C.sha(gpu.q1_apply_resident(h, x, C.D, C.D // 128, 16)) == GOLDEN["c1"]["out_sha256"]


def test_c2_layer_decode_golden(gpu):
    import torch
    layer, cos, sin, kc, vc, x_in = C.c2_inputs()
    net = _net(gpu, {"layers": [layer], "cos": cos, "sin": sin}, 1, C.C2_CTX + 8)
    try:
        net.seed(0, kc[None], vc[None])
        x = torch.from_numpy(x_in.copy()).cuda()
        assert net.forward(x, [C.C2_CTX], 1) == 0
        k, v = net.export_kv(0, 0, C.C2_CTX + 1)
        g = GOLDEN["c2"]
        assert C.sha(x.cpu().numpy()) == g["out_sha256"]
        assert C.sha(k[:, C.C2_CTX:]) == g["k_new_sha256"] and C.sha(v[:, C.C2_CTX:]) == g["v_new_sha256"]
    finally:
        net.close()


def test_c3_layer_prefill_2048_golden(gpu):
    import torch
    layer, cos, sin, x0 = C.c3_inputs()
    T = C.C3_T
    net = _net(gpu, {"layers": [layer], "cos": cos, "sin": sin}, 1, T + 64)
    try:
        x = torch.from_numpy(x0.copy()).cuda()
        assert net.forward(x, [0], T) == 0
        k, v = net.export_kv(0, 0, T)
        g = GOLDEN["c3"]
        assert C.sha(x.cpu().numpy()) == g["out_sha256"], "layer output"
        assert C.sha(k) == g["k_sha256"] and C.sha(v) == g["v_sha256"], "cached K/V rows"
    finally:
        net.close()


def test_c4_moe_golden(gpu):
    from integer_inference_engine_amd import qk_gpu
    c = C.C4
    d, e_ffn = c["d"], c["e_ffn"]
    ex, h, sel, gates = C.c4_inputs()
    hs = [dict(gate=qk_gpu.register_weight(x["gate"], e_ffn, d // 256, 0),
               up=qk_gpu.register_weight(x["up"], e_ffn, d // 256, 0),
               down=qk_gpu.register_weight(x["down"], d, e_ffn // 256, 1)) for x in ex]
    flat = sel.reshape(-1)
    try:
        got = qk_gpu.moe_ffn_batched([hs[e]["gate"] for e in flat], [hs[e]["up"] for e in flat],
                                     [hs[e]["down"] for e in flat], c["T"], c["k"], h, gates, d, e_ffn, 16, 24)
        assert C.sha(got) == GOLDEN["c4"]["out_sha256"]
    finally:
        qk_gpu.free_all()


@pytest.mark.timeout(900)
def test_c5_full_batch_64_steps_golden(gpu):
    import torch
    g = GOLDEN.get("c5")
    if g is None:
        pytest.skip("C5 golden not generated (tests/golden/make_config_golden.py --c5)")
    lens, first, ctx = C.c5_spec()
    B, steps = C.C5["B"], C.C5["steps"]
    model = C.c5_model()
    net = _net(gpu, model, B, 64, with_head=True, n_layers=C.C5["n_layers"])
    eb = torch.from_numpy(np.ascontiguousarray(model["embed"][0])).cuda()
    es = torch.from_numpy(np.ascontiguousarray(model["embed"][1])).cuda()
    del model
    try:
        net.set_caps(lens + steps + 1)
        want_tok = np.array(g["tokens"], dtype=np.int64).T                 # (steps, B)
        # graph-replayed run: every token
        net.fill_kv(C.C5["seed"], lens)
        ids = torch.from_numpy(first.copy()).cuda()
        net.clear_status()
        _, hist = net.decode(eb, es, ids, steps, graph=True)
        assert net.status() == 0
        net.stream.synchronize()
        got_tok = hist.cpu().numpy()
        bad = np.argwhere(got_tok != want_tok)
        assert bad.size == 0, f"{len(bad)} tokens differ, first (step, seq) {bad[0].tolist()}"
        # eager step-by-step rerun: per-step logits digests
        net.reset()
        net.fill_kv(C.C5["seed"], lens)
        ids = torch.from_numpy(first.copy()).cuda()
        logits = torch.empty((B, C.VOCAB), dtype=torch.int64, device="cuda")
        for s in range(steps):
            net.decode(eb, es, ids, 1, graph=False, logits=logits)
            net.stream.synchronize()
            rows = logits.cpu().numpy()
            dig = C.c5_step_digest([hashlib.sha256(rows[b].astype("<i8").tobytes()).hexdigest() for b in range(B)])
            assert dig == g["step_sha256"][s], f"step {s} logits"
            assert np.array_equal(ids.cpu().numpy(), want_tok[s]), f"step {s} tokens (eager)"
        assert net.status() == 0
    finally:
        net.close()
