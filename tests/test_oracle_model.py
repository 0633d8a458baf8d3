"""Structural identities of the oracle's layer graph (CPU only): a causal prefill over T tokens equals T single-token
decodes byte for byte (outputs and the cached K/V), and the batched ragged decode equals per-sequence decodes. The
reference relies on the same identities (prefill-then-decode vs decode-only paths, reference_bonsai.py:941-966,
:1175-1199); a wrong causal mask, RoPE position or cache append breaks them."""
import numpy as np

from oracle import bonsai_model as obm, prng, workloads
from oracle.q1 import q1_rows


def _cfg(model):
    c = model["cfg"]
    return {"H": c["H"], "Hkv": c["Hkv"], "hd": c["hd"]}


def test_prefill_equals_token_by_token_decode():
    model = workloads.small_bonsai(seed=3, ctx=64)
    c = _cfg(model)
    ids = prng.uniform_int(3, 1, (9,), 0, model["cfg"]["vocab"])
    x = q1_rows(*model["embed"], ids)
    for layer in model["layers"]:
        full, kf, vf = obm.layer_forward(x, layer, c, model["cos"], model["sin"], 16, None, None, 0)
        k = v = None
        rows = []
        for t in range(x.shape[0]):
            y, kn, vn = obm.layer_forward(x[t:t + 1], layer, c, model["cos"], model["sin"], 16, k, v, t)
            k = kn if k is None else np.concatenate([k, kn], axis=1)
            v = vn if v is None else np.concatenate([v, vn], axis=1)
            rows.append(y)
        assert np.array_equal(np.concatenate(rows), full)
        assert np.array_equal(k, kf) and np.array_equal(v, vf)
        x = full


def test_batched_ragged_decode_equals_per_sequence():
    model = workloads.small_bonsai(seed=4, ctx=64)
    c = _cfg(model)
    layer = model["layers"][0]
    lens = [3, 11, 6]
    caches = [workloads.kv_fill(4, 10 + b, c["Hkv"], L, c["hd"], mag=1 << 16) for b, L in enumerate(lens)]
    x = prng.uniform_int(4, 2, (3, model["cfg"]["d"]), -(1 << 18), 1 << 18)
    got, kb, vb = obm.layer_decode_batched(x, layer, c, model["cos"], model["sin"], 16,
                                           [k for k, _ in caches], [v for _, v in caches], lens)
    for b, L in enumerate(lens):
        want, kn, vn = obm.layer_forward(x[b:b + 1], layer, c, model["cos"], model["sin"], 16, caches[b][0],
                                         caches[b][1], L)
        assert np.array_equal(got[b:b + 1], want)
        assert np.array_equal(kb[b], kn[:, 0]) and np.array_equal(vb[b], vn[:, 0])


def test_head_rmsnorm_is_rowwise_rmsnorm():
    from oracle import fixedpoint as fx
    xh = prng.uniform_int(5, 1, (4, 3, 32), -(1 << 20), 1 << 20)
    g = prng.uniform_int(5, 2, (32,), 1 << 15, 1 << 17)
    out = obm.head_rmsnorm(xh, 16, g)
    for a in range(4):
        for b in range(3):
            assert np.array_equal(out[a, b], fx.rmsnorm(xh[a, b][None], 16, 1, g)[0])


def test_rowbuf_layer_equals_layer_forward():
    """The in-place row-buffer form (used for 32K-position decodes) equals layer_forward: a 5-row prefill and two
    single-row decodes, outputs and the cache rows, with the C silu/attention restatements."""
    from oracle import c_oracle
    model = workloads.small_bonsai(seed=8, ctx=64)
    c = _cfg(model)
    cfg = model["cfg"]
    ids = prng.uniform_int(8, 1, (7,), 0, cfg["vocab"])
    x = q1_rows(*model["embed"], ids)
    layer = model["layers"][1]
    kb = np.zeros((cfg["Hkv"], 20, cfg["hd"]), dtype=np.int64)
    vb = np.zeros_like(kb)
    k = v = None
    for start, M in ((0, 5), (5, 1), (6, 1)):
        want, kn, vn = obm.layer_forward(x[start:start + M], layer, c, model["cos"], model["sin"], 16, k, v, start)
        k = kn if k is None else np.concatenate([k, kn], axis=1)
        v = vn if v is None else np.concatenate([v, vn], axis=1)
        got = obm.layer_forward_rowbuf(x[start:start + M], layer, c, model["cos"], model["sin"], 16, kb, vb, start,
                                       silu_mul=c_oracle.silu_mul)
        assert np.array_equal(got, want)
        assert np.array_equal(kb[:, :start + M], k) and np.array_equal(vb[:, :start + M], v)
