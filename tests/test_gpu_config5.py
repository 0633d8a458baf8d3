"""Config 5 path: ragged batch decode over a paged, device-filled kv8 cache with the full LM head and greedy argmax.

* exact: 8B-shape layers (3 of them), 4 ragged sequences crossing page boundaries, 4 greedy steps, every token and
  the last logits equal to the oracle's (reference flow: reference_bonsai.py:1175-1199 batched decode, :790-827).
* full depth: 36 layers x 32 sequences with ragged contexts; sequences decoded inside the batch equal the same
  sequences decoded alone (batch invariance), and a replay is identical (determinism).
"""
import numpy as np
import pytest

from oracle import bonsai_model as obm, c_oracle, fixedpoint as fx, prng, q1 as oq1, workloads
from oracle.rope import bonsai8b_tables
from tests.bonsai_gpu_harness import register_model

pytestmark = pytest.mark.gpu
D, H, HKV, HD, DFF, VOCAB = 4096, 32, 8, 128, 12288, 151936
CFG = {"H": H, "Hkv": HKV, "hd": HD}


def _model(n_layers, ctx, seed=12):
    layers = [workloads.bonsai_layer(seed, D, H, HKV, HD, DFF, li) for li in range(n_layers)]
    cos, sin = bonsai8b_tables(ctx)
    return {"layers": layers, "cos": cos, "sin": sin, "embed": workloads.q1_weight(seed, 7, VOCAB, D),
            "out": workloads.q1_weight(seed, 9, VOCAB, D),
            "final_g": prng.uniform_int(seed, 11, (D,), 1 << 15, (1 << 17) + 1)}


def _net(gpu, model, B, caps):
    import torch
    from integer_inference_engine_amd.resident import ResidentNet
    w, g = register_model(gpu, model, with_head=True)
    net = ResidentNet(B=B, n_layers=len(model["layers"]), H=H, Hkv=HKV, hd=HD, d=D, dff=DFF, cap=max(caps), w=w,
                      g=g, page=64, kv32=True)
    net.set_caps(caps)
    eb = torch.from_numpy(np.ascontiguousarray(model["embed"][0])).cuda()
    es = torch.from_numpy(np.ascontiguousarray(model["embed"][1])).cuda()
    return net, eb, es


@pytest.mark.timeout(600)
def test_c5_ragged_batch_exact(gpu):
    import torch
    lens, steps, seed = [5, 63, 81, 200], 4, 5
    model = _model(3, max(lens) + steps + 8)
    first = [11, 2024, 77, 151935]
    net, eb, es = _net(gpu, model, len(lens), [n + steps + 1 for n in lens])
    try:
        net.fill_kv(seed, lens)
        ids = torch.tensor(first, dtype=torch.int64, device="cuda")
        net.clear_status()
        logits, hist = net.decode(eb, es, ids, steps, graph=True)
        assert net.status() == 0
        net.stream.synchronize()
        got_tok = hist.cpu().numpy()
        got_last = logits.cpu().numpy()
    finally:
        net.close()
    for b, L0 in enumerate(lens):
        caches = [(workloads.kv_fill_seq(seed, li, 0, b, HKV, L0, HD), workloads.kv_fill_seq(seed, li, 1, b, HKV, L0, HD))
                  for li in range(len(model["layers"]))]
        tok = first[b]
        for s in range(steps):
            x = oq1.q1_rows(*model["embed"], np.array([tok]))
            for li, layer in enumerate(model["layers"]):
                k, v = caches[li]
                x, kn, vn = obm.layer_forward(x, layer, CFG, model["cos"], model["sin"], 16, k, v, L0 + s,
                                              q1=c_oracle.q1_linear)
                caches[li] = (np.concatenate([k, kn], axis=1), np.concatenate([v, vn], axis=1))
            lg = c_oracle.q1_linear(fx.rmsnorm(x, 16, 1, model["final_g"]), *model["out"], 16)[0]
            tok = int(oq1.argmax_lowest(lg)[0])
            assert got_tok[s, b] == tok, (b, s)
        assert np.array_equal(got_last[b], lg), f"sequence {b}: last logits differ"


@pytest.mark.timeout(900)
def test_c5_full_depth_batch_invariance_and_determinism(gpu):
    import torch
    B, steps, seed = 32, 8, 9
    lens = [int(v) for v in prng.uniform_int(seed, 1, (B,), 64, 2049)]
    model = _model(36, max(lens) + steps + 8, seed=13)
    first = [int(v) for v in prng.uniform_int(seed, 2, (B,), 0, VOCAB)]
    caps = [n + steps + 1 for n in lens]
    runs = []
    net, eb, es = _net(gpu, model, B, caps)
    try:
        for _ in range(2):
            net.set_caps(caps)
            net.fill_kv(seed, lens)
            ids = torch.tensor(first, dtype=torch.int64, device="cuda")
            net.clear_status()
            logits, hist = net.decode(eb, es, ids, steps, graph=True)
            assert net.status() == 0
            net.stream.synchronize()
            runs.append((hist.cpu().numpy(), logits.cpu().numpy()))
    finally:
        net.close()
    assert np.array_equal(runs[0][0], runs[1][0]) and np.array_equal(runs[0][1], runs[1][1]), "replay differs"
    for b in (0, int(np.argmax(lens)), B - 1):
        solo, eb1, es1 = _net(gpu, model, 1, [caps[b]])
        try:
            solo.fill_kv(seed, [lens[b]], seq_ids=[b])
            ids = torch.tensor([first[b]], dtype=torch.int64, device="cuda")
            logits, hist = solo.decode(eb1, es1, ids, steps, graph=True)
            solo.stream.synchronize()
            assert np.array_equal(hist.cpu().numpy()[:, 0], runs[0][0][:, b]), f"sequence {b} tokens"
            assert np.array_equal(logits.cpu().numpy()[0], runs[0][1][b]), f"sequence {b} logits"
        finally:
            solo.close()
