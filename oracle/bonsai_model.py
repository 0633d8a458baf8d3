"""Qwen3-dense Bonsai layer / model forward over packed Q1_0 weights, restated (test infrastructure).

Follows ``bonsai/src/trinote/infer_int/reference_bonsai.py``: ``_run_layers`` (:941-966), cached attention
(:656-720), ``_ffn_ref`` (:603-615), ``_head_rmsnorm`` (:286-297), batched decode (:723-778, :1175-1199) and the
output head + lowest-index argmax (:790-827). ``q1`` is pluggable so the same graph runs with the numpy Q1 oracle
or the C restatement (``oracle.c_oracle``) at large sizes.

Pinned by composition: every primitive is pinned in its own module; the graph itself is checked against the
reference's structure by the per-layer KV-byte and call-count identities in ``tests/test_oracle_model.py``
(prefill over T tokens == T single-token decodes, byte for byte).
"""
from __future__ import annotations

import numpy as np

from . import fixedpoint as fx
from .attention import attention_cached
from .q1 import q1_linear, q1_rows
from .rope import apply_neox, apply_neox_rows

PROJ = ("wq", "wk", "wv", "wo", "w1", "wu", "w2")


def head_rmsnorm(xh: np.ndarray, frac: int, gain: np.ndarray) -> np.ndarray:
    a, b, d = xh.shape
    return fx.rmsnorm(xh.reshape(a * b, d), frac, 1, gain).reshape(a, b, d)


def _silu_mul(gate, up, frac):
    return fx.mulshift_wrap(fx.silu_wrap(gate, frac), up, frac)


def layer_forward(x, layer, cfg, cos, sin, frac, kcache, vcache, start, q1=q1_linear, attn=attention_cached,
                  silu_mul=_silu_mul):
    """One layer over M new positions [start, start+M). kcache/vcache (Hkv, start, hd) or None.
    Returns (x_out (M,d), k_new (Hkv,M,hd) post-norm+RoPE, v_new (Hkv,M,hd)). ``attn`` is pluggable like ``q1``
    (the C restatement ``oracle.c_oracle.attention_cached`` for 2048-token prefills), and so is the FFN's
    SiLU(gate)·up (``oracle.c_oracle.silu_mul``)."""
    M = x.shape[0]
    H, Hkv, hd = cfg["H"], cfg["Hkv"], cfg["hd"]
    n1 = fx.rmsnorm(x, frac, 1, layer["n1g"])
    q = q1(n1, *layer["wq"], frac)
    k = q1(n1, *layer["wk"], frac)
    v = q1(n1, *layer["wv"], frac)
    qh = head_rmsnorm(q.reshape(M, H, hd).transpose(1, 0, 2), frac, layer["qng"])
    kh = head_rmsnorm(k.reshape(M, Hkv, hd).transpose(1, 0, 2), frac, layer["kng"])
    vh = np.ascontiguousarray(v.reshape(M, Hkv, hd).transpose(1, 0, 2))
    qh = apply_neox(qh, cos[start:start + M], sin[start:start + M], frac)
    kh = apply_neox(kh, cos[start:start + M], sin[start:start + M], frac)
    K = kh if kcache is None else np.concatenate([kcache, kh], axis=1)
    V = vh if vcache is None else np.concatenate([vcache, vh], axis=1)
    att = attn(qh, K, V, start, frac, fx.inv_sqrt_fp(hd, frac))
    x = fx.add_wrap(x, q1(att.transpose(1, 0, 2).reshape(M, H * hd), *layer["wo"], frac))
    n2 = fx.rmsnorm(x, frac, 1, layer["n2g"])
    gate = q1(n2, *layer["w1"], frac)
    up = q1(n2, *layer["wu"], frac)
    h = silu_mul(gate, up, frac)
    x = fx.add_wrap(x, q1(h, *layer["w2"], frac))
    return x, kh, vh


def layer_forward_rowbuf(x, layer, cfg, cos, sin, frac, kbuf, vbuf, start, q1=q1_linear, silu_mul=_silu_mul):
    """``layer_forward`` over M new positions [start, start+M) with the cache held in preallocated row buffers
    kbuf/vbuf (Hkv, cap, hd) int64 (rows [0, start) filled): the new post-RoPE K and raw V rows are written in
    place and attention runs over rows [0, start+M) with the C restatement (oracle.c_oracle.attention_ld), so a
    32K-position decode appends without copying the cache. Returns x_out (M, d)."""
    from .c_oracle import attention_ld
    M = x.shape[0]
    H, Hkv, hd = cfg["H"], cfg["Hkv"], cfg["hd"]
    n1 = fx.rmsnorm(x, frac, 1, layer["n1g"])
    qh = head_rmsnorm(q1(n1, *layer["wq"], frac).reshape(M, H, hd).transpose(1, 0, 2), frac, layer["qng"])
    kh = head_rmsnorm(q1(n1, *layer["wk"], frac).reshape(M, Hkv, hd).transpose(1, 0, 2), frac, layer["kng"])
    vh = q1(n1, *layer["wv"], frac).reshape(M, Hkv, hd).transpose(1, 0, 2)
    qh = apply_neox(qh, cos[start:start + M], sin[start:start + M], frac)
    kbuf[:, start:start + M] = apply_neox(kh, cos[start:start + M], sin[start:start + M], frac)
    vbuf[:, start:start + M] = vh
    att = attention_ld(qh, kbuf, vbuf, start + M, start, frac, fx.inv_sqrt_fp(hd, frac))
    x = fx.add_wrap(x, q1(att.transpose(1, 0, 2).reshape(M, H * hd), *layer["wo"], frac))
    n2 = fx.rmsnorm(x, frac, 1, layer["n2g"])
    h = silu_mul(q1(n2, *layer["w1"], frac), q1(n2, *layer["wu"], frac), frac)
    return fx.add_wrap(x, q1(h, *layer["w2"], frac))


def layer_decode_batched(x, layer, cfg, cos, sin, frac, kcaches, vcaches, positions, q1=q1_linear):
    """One decode step for B sequences, row b at absolute position positions[b] with its own cache
    (Hkv, L_b, hd). Rows are independent, so this equals B separate ``layer_forward`` calls."""
    B = x.shape[0]
    H, Hkv, hd = cfg["H"], cfg["Hkv"], cfg["hd"]
    n1 = fx.rmsnorm(x, frac, 1, layer["n1g"])
    q = q1(n1, *layer["wq"], frac)
    k = q1(n1, *layer["wk"], frac)
    v = q1(n1, *layer["wv"], frac)
    qh = head_rmsnorm(q.reshape(B, H, hd), frac, layer["qng"])
    kh = head_rmsnorm(k.reshape(B, Hkv, hd), frac, layer["kng"])
    vh = v.reshape(B, Hkv, hd)
    pos = np.asarray(positions, dtype=np.int64)
    qh = apply_neox_rows(qh, cos[pos], sin[pos], frac)
    kh = apply_neox_rows(kh, cos[pos], sin[pos], frac)
    att = np.empty((B, H, hd), dtype=np.int64)
    k_new, v_new = [], []
    for b in range(B):
        K = np.concatenate([kcaches[b], kh[b][:, None, :]], axis=1)
        V = np.concatenate([vcaches[b], vh[b][:, None, :]], axis=1)
        att[b] = attention_cached(qh[b][:, None, :], K, V, int(pos[b]), frac, fx.inv_sqrt_fp(hd, frac))[:, 0, :]
        k_new.append(kh[b]); v_new.append(vh[b])
    x = fx.add_wrap(x, q1(att.reshape(B, H * hd), *layer["wo"], frac))
    n2 = fx.rmsnorm(x, frac, 1, layer["n2g"])
    h = fx.mulshift_wrap(fx.silu_wrap(q1(n2, *layer["w1"], frac), frac), q1(n2, *layer["wu"], frac), frac)
    x = fx.add_wrap(x, q1(h, *layer["w2"], frac))
    return x, k_new, v_new


def embed(model, ids) -> np.ndarray:
    return q1_rows(model["embed"][0], model["embed"][1], ids)


def head_logits(model, x, frac, q1=q1_linear) -> np.ndarray:
    xn = fx.rmsnorm(x, frac, 1, model["final_g"])
    return q1(xn, *model["out"], frac)
