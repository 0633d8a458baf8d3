"""Single-sequence decode, where every projection builds its digit table in its own prologue (RMSNorm into q/k/v
and gate/up, the attention output into wo, SiLU * up into the down projection): logits, tokens and caches against
the oracle, byte for byte (reference flow: reference_bonsai.py:1200-1310), on shapes whose K is a partial slab,
a ragged number of slabs and the 8B widths, plus the RMSNorm refusals on this path."""
import ctypes

import numpy as np
import pytest

from oracle import bonsai_model as obm, c_oracle, fixedpoint as fx, prng, workloads
from oracle.q1 import q1_rows
from tests.bonsai_gpu_harness import register_model

pytestmark = pytest.mark.gpu

# (d, H, Hkv, hd, dff): d = 128 is one partial 512-slab; 2560 is five slabs (ragged slab ranges) with dff 6912 =
# 13.5 slabs; 4096 / 12288 are the 8B widths (the q/k/v and gate/up launches clear each other's outputs)
SHAPES = [(128, 4, 2, 32, 256), (2560, 4, 2, 128, 6912), (4096, 8, 2, 128, 12288)]


def _model(seed, shape, ctx=64):
    d, H, Hkv, hd, dff = shape
    return workloads.bonsai_model(seed, d=d, H=H, Hkv=Hkv, hd=hd, dff=dff, n_layers=2, vocab=512, ctx=ctx)


def _prefill(model, ids):
    cfg = model["cfg"]
    c = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    x = q1_rows(*model["embed"], ids)
    ks, vs = [], []
    for layer in model["layers"]:
        x, kn, vn = obm.layer_forward(x, layer, c, model["cos"], model["sin"], 16, None, None, 0,
                                        q1=c_oracle.q1_linear)
        ks.append(kn)
        vs.append(vn)
    return x, ks, vs


def _ctx(gpu, model, w, g):
    cfg = model["cfg"]
    ctx = gpu.decode_ctx_create((1, cfg["n_layers"], cfg["H"], cfg["Hkv"], cfg["hd"], cfg["d"], cfg["dff"],
                                 cfg["vocab"]), w, g, 16, 1, fx.inv_sqrt_fp(cfg["hd"], 16), 64)
    assert ctx is not None
    return ctx


@pytest.mark.parametrize("shape", SHAPES)
def test_single_sequence_decode_steps_match_oracle(gpu, shape):
    model = _model(60 + shape[0] % 97, shape)
    cfg = model["cfg"]
    c = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    print(f"[prologue] shape {shape}", flush=True)
    w, g = register_model(gpu, model)
    ctx = _ctx(gpu, model, w, g)
    try:
        prompt = prng.uniform_int(61, 1, (5,), 0, cfg["vocab"])
        x, ks, vs = _prefill(model, prompt)
        assert gpu.decode_ctx_seed_seq(ctx, 0, np.stack(ks), np.stack(vs))
        tok, pos = int(np.argmax(obm.head_logits(model, x[-1:], 16)[0])), len(prompt)
        for step in range(4):
            x_in = q1_rows(*model["embed"], [tok])
            got = gpu.decode_step(ctx, x_in, [pos], cfg["vocab"])
            xb = x_in
            for li, layer in enumerate(model["layers"]):
                xb, kn, vn = obm.layer_forward(xb, layer, c, model["cos"], model["sin"], 16, ks[li], vs[li], pos,
                                               q1=c_oracle.q1_linear)
                ks[li] = np.concatenate([ks[li], kn], axis=1)
                vs[li] = np.concatenate([vs[li], vn], axis=1)
            want = obm.head_logits(model, xb, 16)[0]
            assert got is not None, f"step {step}: refused"
            bad = np.flatnonzero(got[0] != want)
            assert bad.size == 0, f"step {step}: {bad.size} logits differ, first at {bad[0]}"
            tok, pos = int(np.argmax(want)), pos + 1
    finally:
        gpu.decode_ctx_free(ctx)


@pytest.mark.parametrize("graph", [0, 1])
def test_single_sequence_device_decode_graph_replays(gpu, graph):
    """imie_net_decode_dev at B = 1: the captured step (prologue launches included) replayed for steps 2.., every
    token and the last logits row against the oracle's greedy continuation."""
    import torch
    from integer_inference_engine_amd import _lib
    model = _model(62, SHAPES[1])
    cfg = model["cfg"]
    c = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    w, g = register_model(gpu, model)
    ctx = _ctx(gpu, model, w, g)
    steps = 5
    try:
        prompt = prng.uniform_int(62, 1, (7,), 0, cfg["vocab"])
        x, ks, vs = _prefill(model, prompt)
        assert gpu.decode_ctx_seed_seq(ctx, 0, np.stack(ks), np.stack(vs))
        first = int(np.argmax(obm.head_logits(model, x[-1:], 16)[0]))
        want_tok, nxt, pos = [], first, len(prompt)
        for _ in range(steps):
            xb = q1_rows(*model["embed"], [nxt])
            for li, layer in enumerate(model["layers"]):
                xb, kn, vn = obm.layer_forward(xb, layer, c, model["cos"], model["sin"], 16, ks[li], vs[li], pos,
                                               q1=c_oracle.q1_linear)
                ks[li] = np.concatenate([ks[li], kn], axis=1)
                vs[li] = np.concatenate([vs[li], vn], axis=1)
            last = obm.head_logits(model, xb, 16)[0]
            nxt = int(np.argmax(last))
            want_tok.append(nxt)
            pos += 1
        so = _lib.lib()
        eb = torch.from_numpy(np.ascontiguousarray(model["embed"][0])).cuda()
        es = torch.from_numpy(np.ascontiguousarray(model["embed"][1])).cuda()
        ids = torch.tensor([first], dtype=torch.int64, device="cuda")
        lg = torch.empty((1, cfg["vocab"]), dtype=torch.int64, device="cuda")
        hist = torch.full((steps, 1), -1, dtype=torch.int64, device="cuda")
        s = torch.cuda.Stream()
        sp = ctypes.c_void_p(s.cuda_stream)
        so.imie_net_status(ctx, 1, sp)
        rc = so.imie_net_decode_dev(ctx, ctypes.c_void_p(eb.data_ptr()), ctypes.c_void_p(es.data_ptr()),
                                    ctypes.c_void_p(ids.data_ptr()), ctypes.c_void_p(lg.data_ptr()),
                                    ctypes.c_void_p(hist.data_ptr()), steps, graph, sp)
        assert rc == 0, _lib.last_error()
        assert so.imie_net_status(ctx, 0, sp) == 0
        s.synchronize()
        assert hist.cpu().numpy()[:, 0].tolist() == want_tok
        assert np.array_equal(lg.cpu().numpy()[0], last)
    finally:
        gpu.decode_ctx_free(ctx)


@pytest.mark.parametrize("which", ["n1g", "n2g"])
def test_single_sequence_norm_envelope_refused(gpu, which):
    """A gain with max|n| * max|g| beyond int64 (the oracle raises, fixedpoint.py:31-71): the step is refused
    with the RMSNorm code, from either prologue (attention norm or MLP norm)."""
    model = _model(63, SHAPES[0])
    cfg = model["cfg"]
    layer = model["layers"][1]
    layer[which] = np.full_like(layer[which], 1 << 62)
    c = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    x_in = q1_rows(*model["embed"], [3])
    with pytest.raises(OverflowError):
        xb = x_in
        for li, lay in enumerate(model["layers"]):
            xb, _, _ = obm.layer_forward(xb, lay, c, model["cos"], model["sin"], 16, None, None, 0)
    w, g = register_model(gpu, model)
    ctx = _ctx(gpu, model, w, g)
    try:
        from integer_inference_engine_amd import _lib
        x = np.ascontiguousarray(x_in, dtype=np.int64)
        pos = np.zeros(1, dtype=np.int64)
        out = np.empty((1, cfg["vocab"]), dtype=np.int64)
        rc = _lib.lib().bonsai_decode_step(int(ctx), x.ctypes.data, pos.ctypes.data, out.ctypes.data)
        assert rc == 4, rc
    finally:
        gpu.decode_ctx_free(ctx)
