"""Fused kv8 prefill attention on head layouts the 8B shape does not use, through the resident forward
(imie_net_forward_dev, kv8 cache), byte for byte against the oracle layer stack (reference flow:
reference_bonsai.py:542-778):

* one query head per kv head, eight per kv head, and four at head dims 64, 96 and 128 (head dim 128 takes the
  32-bit two-launch form, the others the general one);
* a fresh 150-row prompt (rows 16-tiles, the last one partial, and 64-key steps past the diagonal), and two
  ragged sequences continuing seeded caches of 40 and 200 positions with 33 new rows each.
"""
import numpy as np
import pytest

from oracle import bonsai_model as obm, c_oracle, prng, workloads
from oracle.q1 import q1_rows
from tests.bonsai_gpu_harness import register_model

pytestmark = pytest.mark.gpu

CAP = 320
# (H, Hkv, hd)
LAYOUTS = [(4, 4, 64), (16, 2, 96), (8, 1, 128), (8, 8, 128), (8, 2, 128)]


def _net(gpu, model, B):
    from integer_inference_engine_amd.resident import ResidentNet
    cfg = model["cfg"]
    w, g = register_model(gpu, model, with_head=False)
    return ResidentNet(B=B, n_layers=cfg["n_layers"], H=cfg["H"], Hkv=cfg["Hkv"], hd=cfg["hd"], d=cfg["d"],
                       dff=cfg["dff"], cap=CAP, w=w, g=g, kv32=True)


def _oracle(model, c, x, kc, vc, start):
    nk, nv = [], []
    for li, layer in enumerate(model["layers"]):
        x, k1, v1 = obm.layer_forward(x, layer, c, model["cos"], model["sin"], 16,
                                      kc[li] if kc else None, vc[li] if vc else None, start, q1=c_oracle.q1_linear)
        nk.append(k1)
        nv.append(v1)
    return x, nk, nv


@pytest.mark.parametrize("layout", LAYOUTS)
def test_kv8_prefill_layouts_match_oracle(gpu, layout):
    import torch
    H, Hkv, hd = layout
    seed = 40 + H + 3 * Hkv + hd
    model = workloads.bonsai_model(seed, d=256, H=H, Hkv=Hkv, hd=hd, dff=512, n_layers=2, vocab=64, ctx=CAP)
    cfg = model["cfg"]
    c = {"H": H, "Hkv": Hkv, "hd": hd}
    print(f"[kv8-prefill-shapes] H={H} Hkv={Hkv} hd={hd} fresh", flush=True)
    T = 150
    x0 = q1_rows(*model["embed"], prng.uniform_int(seed, 3, (T,), 0, cfg["vocab"]))
    net = _net(gpu, model, 1)
    try:
        x = torch.from_numpy(x0.copy()).cuda()
        assert net.forward(x, [0], T) == 0
        want, nk, nv = _oracle(model, c, x0, None, None, 0)
        got = x.cpu().numpy()
        assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} outputs differ"
        for li in range(cfg["n_layers"]):
            k, v = net.export_kv(li, 0, T)
            assert np.array_equal(k, nk[li]) and np.array_equal(v, nv[li]), li
    finally:
        net.close()


@pytest.mark.parametrize("layout", LAYOUTS[1:3])
def test_kv8_prefill_layouts_ragged_continued(gpu, layout):
    import torch
    H, Hkv, hd = layout
    seed = 60 + H + 3 * Hkv + hd
    model = workloads.bonsai_model(seed, d=256, H=H, Hkv=Hkv, hd=hd, dff=512, n_layers=2, vocab=64, ctx=CAP)
    cfg = model["cfg"]
    c = {"H": H, "Hkv": Hkv, "hd": hd}
    starts, M = [40, 200], 33
    print(f"[kv8-prefill-shapes] H={H} Hkv={Hkv} hd={hd} ragged {starts} + {M}", flush=True)
    ks = [[prng.uniform_int(seed, 10 + 4 * b + li, (Hkv, starts[b], hd), -(1 << 20), 1 << 20)
           for li in range(cfg["n_layers"])] for b in range(2)]
    vs = [[prng.uniform_int(seed, 12 + 4 * b + li, (Hkv, starts[b], hd), -(1 << 20), 1 << 20)
           for li in range(cfg["n_layers"])] for b in range(2)]
    net = _net(gpu, model, 2)
    try:
        for b in range(2):
            net.seed(b, np.stack(ks[b]), np.stack(vs[b]))
        xs = [q1_rows(*model["embed"], prng.uniform_int(seed, 20 + b, (M,), 0, cfg["vocab"])) for b in range(2)]
        x = torch.from_numpy(np.concatenate(xs)).cuda()
        assert net.forward(x, starts, M) == 0
        got = x.cpu().numpy()
        for b, s0 in enumerate(starts):
            want, nk, nv = _oracle(model, c, xs[b], ks[b], vs[b], s0)
            bad = np.flatnonzero(got[b * M:(b + 1) * M] != want)
            assert bad.size == 0, f"sequence {b}: {bad.size} values differ"
            for li in range(cfg["n_layers"]):
                k, v = net.export_kv(li, b, s0 + M)
                assert np.array_equal(k[:, s0:], nk[li]) and np.array_equal(v[:, s0:], nv[li]), (b, li)
    finally:
        net.close()


def test_kv8_prefill_head128_mixed_launch_paths(gpu):
    """Head dim 128 with one kv head's cached K near 2^26: the query tiles of its 4 heads fail the 32-bit score bound
    (128 max|q| max|K| < 2^47) and are left by the 32-bit launch to the general one, which walks the flagged tiles;
    the other kv head's tiles stay on the 32-bit path. Two ragged sequences continuing seeded caches."""
    import torch
    H, Hkv, hd = 8, 2, 128
    seed = 97
    model = workloads.bonsai_model(seed, d=256, H=H, Hkv=Hkv, hd=hd, dff=512, n_layers=2, vocab=64, ctx=CAP)
    cfg = model["cfg"]
    c = {"H": H, "Hkv": Hkv, "hd": hd}
    starts, M = [50, 130], 40
    print(f"[kv8-prefill-shapes] mixed 32-bit / general tiles {starts} + {M}", flush=True)
    ks, vs = [], []
    for b in range(2):
        kb, vb = [], []
        for li in range(cfg["n_layers"]):
            k = prng.uniform_int(seed, 10 + 4 * b + li, (Hkv, starts[b], hd), -(1 << 20), 1 << 20)
            k[0] = prng.uniform_int(seed, 30 + 4 * b + li, (starts[b], hd), -(1 << 26), 1 << 26)
            kb.append(k)
            vb.append(prng.uniform_int(seed, 12 + 4 * b + li, (Hkv, starts[b], hd), -(1 << 20), 1 << 20))
        ks.append(kb)
        vs.append(vb)
    net = _net(gpu, model, 2)
    try:
        for b in range(2):
            net.seed(b, np.stack(ks[b]), np.stack(vs[b]))
        xs = [q1_rows(*model["embed"], prng.uniform_int(seed, 20 + b, (M,), 0, cfg["vocab"])) for b in range(2)]
        x = torch.from_numpy(np.concatenate(xs)).cuda()
        assert net.forward(x, starts, M) == 0
        got = x.cpu().numpy()
        for b, s0 in enumerate(starts):
            want, nk, nv = _oracle(model, c, xs[b], ks[b], vs[b], s0)
            bad = np.flatnonzero(got[b * M:(b + 1) * M] != want)
            assert bad.size == 0, f"sequence {b}: {bad.size} values differ"
            for li in range(cfg["n_layers"]):
                k, v = net.export_kv(li, b, s0 + M)
                assert np.array_equal(k[:, s0:], nk[li]) and np.array_equal(v[:, s0:], nv[li]), (b, li)
    finally:
        net.close()
