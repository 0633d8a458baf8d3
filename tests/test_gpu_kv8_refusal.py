"""The kv8 cache's range edge on the device. The digit-plane format holds |v| <= 2,139,062,143 = 127·(256^4 − 1)/255
(four balanced int8 digits); the reference's int32-guarded cache refuses anything beyond int32 with a nonzero rc
after an all-lanes preflight (bonsai_q1_gpu.cu:1780-1825, gpu_native.py:218-220). Here:

* seeding (bonsai_decode_ctx_seed_seq) accepts ±2,139,062,143 exactly and refuses ±2,139,062,144, ±(2^31 − 1) and
  −2^31 with rc 2 before writing any cache byte;
* an append through a forward (decode M = 1 and prefill M > 1), with K driven to the edge by the per-head norm gain
  and V by the v projection's scales, is exact at the largest accepted magnitude and sets status bit 2 one step
  beyond it; the refused elements are stored as 0, never as a wrapped value;
* the int64 cache (kv32 = 0) gives the oracle's result for the same out-of-range values.
"""
import numpy as np
import pytest

from oracle import bonsai_model as obm, fixedpoint as fx, prng, workloads
from oracle.q1 import q1_linear, q1_rows
from oracle.rope import apply_neox
from tests.bonsai_gpu_harness import register_model

pytestmark = pytest.mark.gpu

KCAP = 2139062143
EOVF = 2
CTX = 96


def _net(gpu, model, kv32, cap=CTX):
    from integer_inference_engine_amd.resident import ResidentNet
    cfg = model["cfg"]
    w, g = register_model(gpu, model, with_head=False)
    return ResidentNet(B=1, n_layers=cfg["n_layers"], H=cfg["H"], Hkv=cfg["Hkv"], hd=cfg["hd"], d=cfg["d"],
                       dff=cfg["dff"], cap=cap, w=w, g=g, kv32=kv32)


def _oracle(model, x, kcs, vcs, start):
    cfg = model["cfg"]
    c = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    nk, nv = [], []
    for li, layer in enumerate(model["layers"]):
        x, k, v = obm.layer_forward(x, layer, c, model["cos"], model["sin"], 16,
                                    None if kcs is None else kcs[li], None if vcs is None else vcs[li], start)
        nk.append(k)
        nv.append(v)
    return x, nk, nv


def _layer0_kv(model, x, start, kng=None, v_scale_mul=1):
    """Layer 0's new K (post-norm, post-RoPE) and V rows for rows x at positions start.. (oracle arithmetic)."""
    cfg, layer = model["cfg"], model["layers"][0]
    M, Hkv, hd = x.shape[0], cfg["Hkv"], cfg["hd"]
    n1 = fx.rmsnorm(x, 16, 1, layer["n1g"])
    k = q1_linear(n1, *layer["wk"], 16).reshape(M, Hkv, hd).transpose(1, 0, 2)
    kh = obm.head_rmsnorm(k, 16, layer["kng"] if kng is None else kng)
    kh = apply_neox(kh, model["cos"][start:start + M], model["sin"][start:start + M], 16)
    bits, scale = layer["wv"]
    v = q1_linear(n1, bits, scale * v_scale_mul, 16).reshape(M, Hkv, hd).transpose(1, 0, 2)
    return kh, v


def _edge(f, lo, hi):
    """Largest integer a in [lo, hi) with f(a) <= KCAP, given f(lo) <= KCAP < f(hi)."""
    assert f(lo) <= KCAP < f(hi)
    while hi - lo > 1:
        mid = (lo + hi) // 2
        if f(mid) <= KCAP:
            lo = mid
        else:
            hi = mid
    return lo


def _absmax(a):
    return int(np.max(np.abs(a.astype(object)))) if a.size else 0


def _edge_models(seed, x, start):
    """Three variants of the small model: K at the largest accepted |K| (constant head-norm gain), K one gain
    step beyond, V at the edge / beyond (v projection scales times an integer factor)."""
    base = workloads.small_bonsai(seed=seed, ctx=CTX)
    hd = base["cfg"]["hd"]
    fk = lambda c: _absmax(_layer0_kv(base, x, start, kng=np.full(hd, c, dtype=np.int64))[0])
    ck = _edge(fk, 1, 1 << 34)
    fv = lambda m: _absmax(_layer0_kv(base, x, start, v_scale_mul=m)[1])
    mv = _edge(fv, 1, 1 << 24)
    out = {}
    for name, c, m in (("k_edge", ck, 1), ("k_over", ck + 1, 1), ("v_edge", None, mv), ("v_over", None, mv + 1)):
        model = workloads.small_bonsai(seed=seed, ctx=CTX)
        layer = model["layers"][0]
        if c is not None:
            layer["kng"] = np.full(hd, c, dtype=np.int64)
        if m != 1:
            layer["wv"] = (layer["wv"][0], layer["wv"][1] * m)
        out[name] = model
    return out


def _check_append(gpu, model, name, x0, start, kv32, prefix=None):
    import torch
    cfg = model["cfg"]
    net = _net(gpu, model, kv32)
    try:
        if prefix is not None:
            net.seed(0, np.stack(prefix[0]), np.stack(prefix[1]))
        x = torch.from_numpy(x0.copy()).cuda()
        status = net.forward(x, [start], x0.shape[0])
        want, nk, nv = _oracle(model, x0, None if prefix is None else prefix[0],
                               None if prefix is None else prefix[1], start)
        over = _absmax(nk[0]) > KCAP or _absmax(nv[0]) > KCAP
        print(f"[kv8-edge] {name} kv32={kv32} start={start} M={x0.shape[0]} max|K|={_absmax(nk[0])} "
              f"max|V|={_absmax(nv[0])} status={status}", flush=True)
        if over and kv32:
            assert status & EOVF, f"{name}: out-of-range append not refused"
            k, v = net.export_kv(0, 0, start + x0.shape[0])
            for got, ref in ((k, nk[0]), (v, nv[0])):
                new = got[:, start:]
                fits = np.abs(ref) <= KCAP
                assert np.array_equal(new[fits], ref[fits])
                assert not np.any(new[~fits]), f"{name}: a refused element was stored"
            return
        assert status == 0, f"{name}: status {status}"
        assert np.array_equal(x.cpu().numpy(), want), name
        for li in range(cfg["n_layers"]):
            k, v = net.export_kv(li, 0, start + x0.shape[0])
            assert np.array_equal(k[:, start:], nk[li]) and np.array_equal(v[:, start:], nv[li]), (name, li)
    finally:
        net.close()


@pytest.mark.parametrize("M", [1, 5])
def test_append_edge(gpu, M):
    """Decode (M = 1 after a 7-position prefix) and prefill (M = 5 from position 0)."""
    base = workloads.small_bonsai(seed=40 + M, ctx=CTX)
    cfg = base["cfg"]
    start = 7 if M == 1 else 0
    x0 = q1_rows(*base["embed"], prng.uniform_int(40 + M, 1, (M,), 0, cfg["vocab"]))
    prefix = None
    if start:
        ks = [prng.uniform_int(40 + M, 10 + l, (cfg["Hkv"], start, cfg["hd"]), -(1 << 20), 1 << 20)
              for l in range(cfg["n_layers"])]
        vs = [prng.uniform_int(40 + M, 20 + l, (cfg["Hkv"], start, cfg["hd"]), -(1 << 20), 1 << 20)
              for l in range(cfg["n_layers"])]
        prefix = (ks, vs)
    models = _edge_models(40 + M, x0, start)
    for name, model in models.items():
        _check_append(gpu, model, name, x0, start, True, prefix)
    for name in ("k_over", "v_over"):                 # no cap on the int64 cache
        _check_append(gpu, models[name], name, x0, start, False, prefix)


def test_seed_edge(gpu):
    """Seed values at the edge (accepted, exact, and a decode step over them equals the oracle), then values
    beyond it (rc 2, no cache byte written)."""
    import torch
    model = workloads.small_bonsai(seed=61, ctx=CTX)
    cfg = model["cfg"]
    nl, Hkv, hd, L = cfg["n_layers"], cfg["Hkv"], cfg["hd"], 9
    ks = prng.uniform_int(61, 1, (nl, Hkv, L, hd), -(1 << 20), 1 << 20)
    vs = prng.uniform_int(61, 2, (nl, Hkv, L, hd), -(1 << 20), 1 << 20)
    ks[0, 0, 0, 0], ks[0, 1, 3, 5], ks[1, 0, 8, hd - 1] = KCAP, -KCAP, KCAP
    vs[0, 0, 2, 1], vs[1, 1, 4, 7], vs[1, 0, 8, 0] = -KCAP, KCAP, KCAP
    x0 = q1_rows(*model["embed"], prng.uniform_int(61, 3, (1,), 0, cfg["vocab"]))
    for kv32 in (True, False):
        net = _net(gpu, model, kv32)
        try:
            net.seed(0, ks, vs)
            for li in range(nl):
                k, v = net.export_kv(li, 0, L)
                assert np.array_equal(k, ks[li]) and np.array_equal(v, vs[li])
            if kv32:
                for bad in (KCAP + 1, -(KCAP + 1), (1 << 31) - 1, -(1 << 31)):
                    for which in ("k", "v"):
                        k2, v2 = ks.copy(), vs.copy()
                        (k2 if which == "k" else v2)[1, 1, 6, 3] = bad
                        print(f"[kv8-edge] seed {which}={bad}", flush=True)
                        with pytest.raises(RuntimeError, match="rc=2"):
                            net.seed(0, k2, v2)
                        for li in range(nl):             # the refused seed wrote nothing
                            k, v = net.export_kv(li, 0, L)
                            assert np.array_equal(k, ks[li]) and np.array_equal(v, vs[li])
            x = torch.from_numpy(x0.copy()).cuda()
            assert net.forward(x, [L], 1) == 0
            want, _, _ = _oracle(model, x0, list(ks), list(vs), L)
            assert np.array_equal(x.cpu().numpy(), want), f"kv32={kv32}"
        finally:
            net.close()

    # beyond the kv8 range the int64 cache still matches the oracle
    ks[1, 1, 6, 3], vs[0, 1, 1, 2] = (1 << 31) - 1, -(1 << 31)
    net = _net(gpu, model, False)
    try:
        net.seed(0, ks, vs)
        x = torch.from_numpy(x0.copy()).cuda()
        assert net.forward(x, [L], 1) == 0
        want, _, _ = _oracle(model, x0, list(ks), list(vs), L)
        assert np.array_equal(x.cpu().numpy(), want)
    finally:
        net.close()


def test_kv8_refuses_head_dims_off_the_tile(gpu):
    """The tiled K layout needs hd % 16 == 0: a kv8 context with hd = 72 is refused at creation (the int64 cache
    takes it)."""
    model = workloads.bonsai_model(62, d=128, H=16, Hkv=2, hd=72, dff=256, n_layers=1, vocab=64, ctx=CTX)
    with pytest.raises(RuntimeError, match="imie_net_create failed"):
        _net(gpu, model, True)
    _net(gpu, model, False).close()
