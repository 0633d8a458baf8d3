"""Bonsai-8B-shape batch-1 greedy decode through all 36 layers and the 151936-entry Q1_0 LM head, over a
4096-position int32 paged KV cache, against the oracle: every step's logits, argmax token and new KV rows must be
byte-identical (reference flow: reference_bonsai.py:1200-1310 decode loop, :790-827 head + argmax)."""
import numpy as np
import pytest

from oracle import bonsai_model as obm, c_oracle, fixedpoint as fx, prng, q1 as oq1, workloads
from oracle.rope import bonsai8b_tables

D, H, HKV, HD, DFF, CTX, NL, VOCAB, STEPS = 4096, 32, 8, 128, 12288, 4096, 36, 151936, 3
CFG = {"H": H, "Hkv": HKV, "hd": HD}


def _model():
    layers = [workloads.bonsai_layer(8, D, H, HKV, HD, DFF, li) for li in range(NL)]
    cos, sin = bonsai8b_tables(CTX + 64)
    return {"layers": layers, "cos": cos, "sin": sin, "embed": workloads.q1_weight(8, 7, VOCAB, D),
            "out": workloads.q1_weight(8, 9, VOCAB, D), "final_g": prng.uniform_int(8, 11, (D,), 1 << 15, (1 << 17) + 1)}


def _kv():
    return workloads.kv_fill(8, 50, HKV, CTX, HD)


def oracle_decode(model, kc, vc, first_id):
    """Greedy steps at positions CTX, CTX+1, ...; every layer starts from the same seeded cache (kc, vc)."""
    caches = [(kc, vc) for _ in range(NL)]
    tok, out = first_id, []
    for s in range(STEPS):
        x = oq1.q1_rows(*model["embed"], np.array([tok]))
        new_kv = []
        for li, layer in enumerate(model["layers"]):
            k, v = caches[li]
            x, kn, vn = obm.layer_forward(x, layer, CFG, model["cos"], model["sin"], 16, k, v, CTX + s,
                                          q1=c_oracle.q1_linear)
            caches[li] = (np.concatenate([k, kn], axis=1), np.concatenate([v, vn], axis=1))
            new_kv.append((kn, vn))
        logits = c_oracle.q1_linear(fx.rmsnorm(x, 16, 1, model["final_g"]), *model["out"], 16)[0]
        tok = int(oq1.argmax_lowest(logits)[0])
        out.append((logits, tok, new_kv))
    return out


@pytest.mark.gpu
@pytest.mark.timeout(400)
def test_8b_decode_36_layers_byte_exact(gpu):
    import torch
    from integer_inference_engine_amd.resident import ResidentNet
    from tests.bonsai_gpu_harness import register_model
    model = _model()
    kc, vc = _kv()
    print("[decode8b] oracle", flush=True)
    want = oracle_decode(model, kc, vc, 7)
    print("[decode8b] device", flush=True)
    w, g = register_model(gpu, model, with_head=True)
    net = ResidentNet(B=1, n_layers=NL, H=H, Hkv=HKV, hd=HD, d=D, dff=DFF, cap=CTX + 64, w=w, g=g, page=64,
                      kv32=True)
    try:
        net.seed(0, np.broadcast_to(kc, (NL,) + kc.shape), np.broadcast_to(vc, (NL,) + vc.shape))
        eb = torch.from_numpy(np.ascontiguousarray(model["embed"][0])).cuda()
        es = torch.from_numpy(np.ascontiguousarray(model["embed"][1])).cuda()
        ids = torch.tensor([7], dtype=torch.int64, device="cuda")
        net.clear_status()
        logits, hist = net.decode(eb, es, ids, STEPS, graph=True)   # step 1 eager, steps 2.. graph replays
        assert net.status() == 0
        net.stream.synchronize()
        assert hist.cpu().numpy()[:, 0].tolist() == [t for _, t, _ in want]
        got = logits.cpu().numpy()[0]
        wl = want[-1][0]
        assert np.array_equal(got, wl), f"{np.count_nonzero(got != wl)} last-step logits differ"
        for li in (0, NL // 2, NL - 1):
            k, v = net.export_kv(li, 0, CTX + STEPS)
            assert np.array_equal(k[:, :CTX], kc) and np.array_equal(v[:, :CTX], vc)
            for s in range(STEPS):
                assert np.array_equal(k[:, CTX + s:CTX + s + 1], want[s][2][li][0]), (li, s)
                assert np.array_equal(v[:, CTX + s:CTX + s + 1], want[s][2][li][1]), (li, s)
    finally:
        net.close()
