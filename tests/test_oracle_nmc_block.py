"""The nmc decode-step oracle (oracle/nmc_block.py) against a full-sequence restatement of the reference block
(CPU only). The restatement here follows north-mini-code/src/nmc/cohere2.py directly and independently of the
decode form: the boolean mask of :85-92 (future keys, and keys at or older than i - window, disallowed) filled with
the -(1 << (fa + 30)) sentinel before a row softmax over ALL keys (:136-161), the parallel residual
x + Attn(n(x)) + MoE(n(x)) with one shared norm and RoPE only on sliding-window layers (:191-199), and the MoE
(router linear, lowest-index top-k, sigmoid gates, SwiGLU experts, :162-188). The decode form attends only the
visible keys; equality at every position pins its window rule (first key = pos - window + 1) and its composition."""
import numpy as np
import pytest

from oracle import fixedpoint as fx, nmc_block as onb, prng
from oracle.rope import apply_interleaved, build_rope_tables

FA, FW = 16, 24


def _full_attention(q, k, v, window, fa):
    """q (S, H, hd), k/v (S, Hkv, hd) -> (S, H, hd): masked full-sequence form."""
    S, H, hd = q.shape
    rep = H // k.shape[1]
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    mask = j > i if window is None else (j > i) | (j <= i - window)
    inv = int(round((1.0 / np.sqrt(hd)) * (1 << fa)))
    out = np.empty((S, H, hd), dtype=np.int64)
    for h in range(H):
        qh = q[:, h].astype(object)
        kh = k[:, h // rep].astype(object)
        vh = v[:, h // rep].astype(object)
        sc = (((qh @ kh.T) >> fa) * inv) >> fa
        sc = np.asarray(sc, dtype=np.int64)
        sc[mask] = -(1 << (fa + 30))
        p = fx.softmax_rows(sc, fa)
        out[:, h] = ((p.astype(object) @ vh) >> fa).astype(np.int64)
    return out


@pytest.mark.parametrize("window", [None, 1, 3, 6])
def test_attention_step_equals_masked_full_sequence(window):
    S, H, Hkv, hd = 7, 4, 2, 8
    q = prng.uniform_int(5, 1, (S, H, hd), -(1 << 18), 1 << 18)
    k = prng.uniform_int(5, 2, (S, Hkv, hd), -(1 << 18), 1 << 18)
    v = prng.uniform_int(5, 3, (S, Hkv, hd), -(1 << 20), 1 << 20)
    full = _full_attention(q, k, v, window, FA)
    kc = np.ascontiguousarray(k.transpose(1, 0, 2))
    vc = np.ascontiguousarray(v.transpose(1, 0, 2))
    for pos in range(S):
        got = onb.attention_step(q[pos], kc, vc, pos, window, FA, fx.inv_sqrt_fp(hd, FA))
        assert np.array_equal(got, full[pos]), (window, pos)


def _lin(x, W):
    return ((np.atleast_2d(x).astype(object) @ np.asarray(W).astype(object).T) >> FW).astype(np.int64)


def _moe_full(h, router, experts, used):
    """cohere2.moe_layer_int restated: per token the lowest-index top-k of the router logits, sigmoid gates,
    SwiGLU experts, sum of per-expert floors."""
    logits = _lin(h, router)
    out = np.zeros(h.shape, dtype=object)
    for t in range(h.shape[0]):
        sel = np.argsort(-logits[t], kind="stable")[:used]
        gates = fx.sigmoid(logits[t][sel], FA, hard_cap=False)
        for j, e in enumerate(sel):
            g = _lin(h[t], experts[int(e)]["gate"])
            g = ((g.astype(object) * fx.sigmoid(g, FA, hard_cap=False).astype(object)) >> FA).astype(np.int64)
            gu = ((g.astype(object) * _lin(h[t], experts[int(e)]["up"]).astype(object)) >> FA).astype(np.int64)
            out[t] += (_lin(gu, experts[int(e)]["down"])[0].astype(object) * int(gates[j])) >> FA
    return out.astype(np.int64)


@pytest.mark.parametrize("window,rope", [(None, False), (2, True)])
def test_block_step_equals_full_sequence_block(window, rope):
    """moe_block_int of cohere2.py:191-199 over S positions vs block_step at each position with the cache of the
    earlier ones: full-attention layers are NoPE, sliding-window layers rotate q and k (interleaved)."""
    S, d, H, Hkv, hd, E, used, ffn = 5, 32, 4, 2, 8, 6, 2, 16
    cfg = {"fa": FA, "fw": FW, "H": H, "Hkv": Hkv, "hd": hd, "used": used, "eps": 1}
    W = {name: prng.uniform_int(9, i, shape, -(1 << 22), 1 << 22)
         for i, (name, shape) in enumerate((("wq", (H * hd, d)), ("wk", (Hkv * hd, d)), ("wv", (Hkv * hd, d)),
                                            ("wo", (d, H * hd)), ("router", (E, d))))}
    W["gain"] = prng.uniform_int(9, 10, (d,), 1 << 15, 1 << 17)
    experts = {e: {n: prng.uniform_int(9, 20 + 3 * e + i, shape, -(1 << 22), 1 << 22)
                   for i, (n, shape) in enumerate((("gate", (ffn, d)), ("up", (ffn, d)), ("down", (d, ffn))))}
               for e in range(E)}
    x = prng.uniform_int(9, 50, (S, d), -(1 << 18), 1 << 18)
    cos, sin = build_rope_tables(S, hd, 50000.0, FA)
    # full-sequence block
    h = fx.rmsnorm(x, FA, 1, W["gain"])
    q = _lin(h, W["wq"]).reshape(S, H, hd)
    k = _lin(h, W["wk"]).reshape(S, Hkv, hd)
    v = _lin(h, W["wv"]).reshape(S, Hkv, hd)
    if rope:
        q = apply_interleaved(q.transpose(1, 0, 2), cos, sin, FA).transpose(1, 0, 2)
        k = apply_interleaved(k.transpose(1, 0, 2), cos, sin, FA).transpose(1, 0, 2)
    att = _lin(_full_attention(q, k, v, window, FA).reshape(S, H * hd), W["wo"])
    want = x + att + _moe_full(h, W["router"], experts, used)
    # the decode form, one position at a time
    kc = np.zeros((Hkv, S, hd), dtype=np.int64)
    vc = np.zeros_like(kc)
    for pos in range(S):
        out, _, _, _, kn, vn = onb.block_step(x[pos:pos + 1], W, kc, vc, pos, window, rope, cos, sin, cfg, experts)
        kc[:, pos], vc[:, pos] = kn, vn
        assert np.array_equal(out[0], want[pos]), (window, pos)
