"""kv8 decode attention on head layouts the 8B shape does not use, through the resident forward (imie_net_forward_dev,
kv8 cache), byte for byte against the oracle layer stack (reference flow: reference_bonsai.py:542-778):

* one query head per kv head, eight per kv head, and four (the 8B layout) at head dims 64, 96 (a second 64-dim K
  step that is partly past hd) and 128;
* one sequence with a seeded 700-position cache (many key chunks) and two ragged sequences (700 and 131 positions),
  each taking two decode steps.
"""
import numpy as np
import pytest

from oracle import bonsai_model as obm, c_oracle, prng, workloads
from oracle.q1 import q1_rows
from tests.bonsai_gpu_harness import register_model

pytestmark = pytest.mark.gpu

CAP = 768
# (H, Hkv, hd)
LAYOUTS = [(4, 4, 64), (16, 2, 96), (8, 1, 128), (8, 2, 128)]


def _net(gpu, model, B):
    from integer_inference_engine_amd.resident import ResidentNet
    cfg = model["cfg"]
    w, g = register_model(gpu, model, with_head=False)
    return ResidentNet(B=B, n_layers=cfg["n_layers"], H=cfg["H"], Hkv=cfg["Hkv"], hd=cfg["hd"], d=cfg["d"],
                       dff=cfg["dff"], cap=CAP, w=w, g=g, kv32=True)


@pytest.mark.parametrize("lens", [[700], [700, 131]])
@pytest.mark.parametrize("layout", LAYOUTS)
def test_kv8_decode_layouts_match_oracle(gpu, layout, lens):
    import torch
    H, Hkv, hd = layout
    seed = 70 + H + 3 * Hkv + hd + len(lens)
    model = workloads.bonsai_model(seed, d=256, H=H, Hkv=Hkv, hd=hd, dff=512, n_layers=2, vocab=64, ctx=CAP)
    cfg = model["cfg"]
    c = {"H": H, "Hkv": Hkv, "hd": hd}
    B = len(lens)
    print(f"[kv8-shapes] H={H} Hkv={Hkv} hd={hd} lens={lens}", flush=True)
    ks = [[prng.uniform_int(seed, 10 + 4 * b + li, (Hkv, lens[b], hd), -(1 << 20), 1 << 20)
           for li in range(cfg["n_layers"])] for b in range(B)]
    vs = [[prng.uniform_int(seed, 12 + 4 * b + li, (Hkv, lens[b], hd), -(1 << 20), 1 << 20)
           for li in range(cfg["n_layers"])] for b in range(B)]
    net = _net(gpu, model, B)
    try:
        for b in range(B):
            net.seed(b, np.stack(ks[b]), np.stack(vs[b]))
        pos = list(lens)
        ids = prng.uniform_int(seed, 3, (B,), 0, cfg["vocab"])
        for step in range(2):
            x0 = q1_rows(*model["embed"], ids)
            x = torch.from_numpy(x0.copy()).cuda()
            assert net.forward(x, pos, 1) == 0, f"step {step}: refused"
            got = x.cpu().numpy()
            for b in range(B):
                xb = x0[b:b + 1]
                for li, layer in enumerate(model["layers"]):
                    xb, kn, vn = obm.layer_forward(xb, layer, c, model["cos"], model["sin"], 16, ks[b][li],
                                                   vs[b][li], pos[b], q1=c_oracle.q1_linear)
                    ks[b][li] = np.concatenate([ks[b][li], kn], axis=1)
                    vs[b][li] = np.concatenate([vs[b][li], vn], axis=1)
                bad = np.flatnonzero(got[b] != xb[0])
                assert bad.size == 0, f"step {step} seq {b}: {bad.size} values differ, first at {bad[0]}"
            ids = np.array([int(np.sum(got[b]) % cfg["vocab"]) for b in range(B)], dtype=np.int64)
            pos = [p + 1 for p in pos]
    finally:
        net.close()
