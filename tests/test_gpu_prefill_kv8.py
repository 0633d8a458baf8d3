"""Prefill (M > 1 new rows per sequence) over the kv8 digit-plane cache, whose attention runs as int8 MFMAs, vs the
oracle byte for byte: layer outputs and the cached K/V, single and ragged multi-sequence, fresh and continued."""
import numpy as np
import pytest

from oracle import bonsai_model as obm, c_oracle, prng, workloads
from oracle.q1 import q1_rows
from oracle.rope import bonsai8b_tables
from tests.bonsai_gpu_harness import register_model

pytestmark = pytest.mark.gpu


def _oracle_layers(model, x, cfgc, kcs, vcs, start):
    """All layers over rows x (M, d) at positions start..; kcs/vcs per-layer caches (Hkv, start, hd) or None."""
    new_k, new_v = [], []
    for li, layer in enumerate(model["layers"]):
        kc = kcs[li] if kcs is not None else None
        vc = vcs[li] if vcs is not None else None
        x, kn, vn = obm.layer_forward(x, layer, cfgc, model["cos"], model["sin"], 16, kc, vc, start,
                                      q1=c_oracle.q1_linear)
        new_k.append(kn)
        new_v.append(vn)
    return x, new_k, new_v


def _net(gpu, model, B, cap, page=64):
    from integer_inference_engine_amd.resident import ResidentNet
    cfg = model["cfg"]
    w, g = register_model(gpu, model, with_head=False)
    return ResidentNet(B=B, n_layers=cfg["n_layers"], H=cfg["H"], Hkv=cfg["Hkv"], hd=cfg["hd"], d=cfg["d"],
                       dff=cfg["dff"], cap=cap, w=w, g=g, page=page, kv32=True)


@pytest.mark.parametrize("T", [2, 17, 64, 100, 256])
def test_small_model_prefill_kv8(gpu, T):
    """T = 256 runs the projections on the +-1 sign-copy GEMM (wo / w2 accumulating into the residual)."""
    import torch
    model = workloads.small_bonsai(seed=50 + T, ctx=320)
    cfg = model["cfg"]
    c = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    ids = prng.uniform_int(T, 5, (T,), 0, cfg["vocab"])
    x0 = q1_rows(*model["embed"], ids)
    net = _net(gpu, model, 1, 320)
    try:
        x = torch.from_numpy(x0.copy()).cuda()
        assert net.forward(x, [0], T) == 0
        got = x.cpu().numpy()
        want, nk, nv = _oracle_layers(model, x0, c, None, None, 0)
        assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} outputs differ"
        for li in range(cfg["n_layers"]):
            k, v = net.export_kv(li, 0, T)
            assert np.array_equal(k, nk[li]) and np.array_equal(v, nv[li]), li
    finally:
        net.close()


def test_ragged_continued_prefill_kv8(gpu):
    """B = 2 sequences with seeded prefixes of 9 and 70 positions, 24 new rows each (causal over prefix + new)."""
    import torch
    model = workloads.small_bonsai(seed=77, ctx=256)
    cfg = model["cfg"]
    c = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    starts, M = [9, 70], 24
    net = _net(gpu, model, 2, 192)
    try:
        pre = []
        for b, s0 in enumerate(starts):
            ids = prng.uniform_int(77, 10 + b, (s0,), 0, cfg["vocab"])
            _, ks, vs = _oracle_layers(model, q1_rows(*model["embed"], ids), c, None, None, 0)
            net.seed(b, np.stack(ks), np.stack(vs))
            pre.append((ks, vs))
        xs = [q1_rows(*model["embed"], prng.uniform_int(77, 20 + b, (M,), 0, cfg["vocab"])) for b in range(2)]
        x = torch.from_numpy(np.concatenate(xs)).cuda()
        assert net.forward(x, starts, M) == 0
        got = x.cpu().numpy()
        for b, s0 in enumerate(starts):
            want, nk, nv = _oracle_layers(model, xs[b], c, pre[b][0], pre[b][1], s0)
            assert np.array_equal(got[b * M:(b + 1) * M], want), f"sequence {b}"
            for li in range(cfg["n_layers"]):
                k, v = net.export_kv(li, b, s0 + M)
                assert np.array_equal(k[:, s0:], nk[li]) and np.array_equal(v[:, s0:], nv[li]), (b, li)
                assert np.array_equal(k[:, :s0], pre[b][0][li]) and np.array_equal(v[:, :s0], pre[b][1][li])
    finally:
        net.close()


def test_8b_layer_prefill_kv8(gpu):
    """One Bonsai-8B-shape layer over a 256-token prompt (config-3 shape at reduced length)."""
    import torch
    D, H, HKV, HD, DFF, T = 4096, 32, 8, 128, 12288, 256
    layer = workloads.bonsai_layer(3, D, H, HKV, HD, DFF)
    cos, sin = bonsai8b_tables(T + 64)
    model = {"layers": [layer], "cos": cos, "sin": sin,
             "cfg": {"n_layers": 1, "H": H, "Hkv": HKV, "hd": HD, "d": D, "dff": DFF}}
    x0 = prng.uniform_int(3, 60, (T, D), -(1 << 20), 1 << 20)
    net = _net(gpu, model, 1, T + 64)
    try:
        x = torch.from_numpy(x0.copy()).cuda()
        assert net.forward(x, [0], T) == 0
        got = x.cpu().numpy()
        want, nk, nv = _oracle_layers(model, x0, {"H": H, "Hkv": HKV, "hd": HD}, None, None, 0)
        assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} outputs differ"
        k, v = net.export_kv(0, 0, T)
        assert np.array_equal(k, nk[0]) and np.array_equal(v, nv[0])
    finally:
        net.close()


def test_kv8_attention_with_wide_queries(gpu):
    """q-norm gains scaled by 2^23 and k-norm gains by 2^-12: q needs 6 limbs, the scores' digit products reach
    exponents >= 8 (which vanish mod 2^64). Prefill of 24 rows, then 3 single-row decode steps over the cache."""
    import torch
    model = workloads.small_bonsai(seed=91, ctx=256)
    for layer in model["layers"]:
        layer["qng"] = (layer["qng"].astype(np.int64) << 23).astype(np.int64)
        layer["kng"] = np.maximum(layer["kng"].astype(np.int64) >> 12, 1)
    cfg = model["cfg"]
    c = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    T = 24
    ids = prng.uniform_int(91, 5, (T + 3,), 0, cfg["vocab"])
    x0 = q1_rows(*model["embed"], ids)
    net = _net(gpu, model, 1, 64)
    try:
        x = torch.from_numpy(x0[:T].copy()).cuda()
        assert net.forward(x, [0], T) == 0
        want, kc, vc = _oracle_layers(model, x0[:T], c, None, None, 0)
        assert np.array_equal(x.cpu().numpy(), want), "prefill"
        for s in range(3):
            xs = torch.from_numpy(x0[T + s:T + s + 1].copy()).cuda()
            assert net.forward(xs, [T + s], 1) == 0
            w1, nk, nv = _oracle_layers(model, x0[T + s:T + s + 1], c, kc, vc, T + s)
            assert np.array_equal(xs.cpu().numpy(), w1), f"decode step {s}"
            kc = [np.concatenate([a, b], axis=1) for a, b in zip(kc, nk)]
            vc = [np.concatenate([a, b], axis=1) for a, b in zip(vc, nv)]
    finally:
        net.close()
