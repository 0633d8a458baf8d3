"""Fixed-point attention, restated (test infrastructure).

Follows the numpy path of ``bonsai/src/trinote/infer_int/reference_bonsai.py``: cached attention ``:656-720``
(scores ``((q K^T) >> f * inv_sqrt) >> f``, causal sentinel ``-(1 << (f + 30))``, softmax, ``(P V) >> f``, both
matmuls fail-loud), prefill ``:586-598`` and batched decode ``:723-778``.

``attention_cached`` raises ``OverflowError`` exactly where the reference raises. The producers' rc-2 rule
(per query row; ``bonsai/tools/bonsai_q1_kernel.c:1466-1500``) is restated separately in ``producer_overflow``.

Pinned by: a per-head big-int brute force (restating ``bonsai/tests/test_bonsai_smoke.py:1563-1576``), key-order
permutation invariance, the compiled reference C kernels (``oracle/_ref``), and the masked-key identity (keys
after the causal limit contribute exactly 0).
"""
from __future__ import annotations

import numpy as np

from . import fixedpoint as fx


def attention_cached(qh: np.ndarray, k: np.ndarray, v: np.ndarray, start: int, frac: int, inv_sqrt: int) -> np.ndarray:
    """qh (H, M, hd) post q-norm+RoPE; k/v (Hkv, L, hd) with L = start + M. Returns (H, M, hd)."""
    H, M, hd = qh.shape
    Hkv, L, _ = k.shape
    assert L == start + M
    rep = H // Hkv
    neg = np.int64(-(1 << (frac + fx.NEG_INF_SHIFT)))
    mask = np.arange(L)[None, :] > (start + np.arange(M))[:, None]
    out = np.empty((H, M, hd), dtype=np.int64)
    with np.errstate(over="ignore"):
        for h in range(H):
            kv = h // rep
            s = fx.fixed_point_matmul(qh[h], k[kv].T, frac)
            s = (s * np.int64(inv_sqrt)) >> np.int64(frac)
            s = np.where(mask, neg, s)
            p = fx.softmax_rows(s, frac)
            out[h] = fx.fixed_point_matmul(p, v[kv], frac)
    return out


def attention_decode_batched(q: np.ndarray, ks, vs, frac: int, inv_sqrt: int) -> np.ndarray:
    """q (B, H, hd); ks[b]/vs[b] (Hkv, L_b, hd). Single query attends all L_b keys (no mask)."""
    B, H, hd = q.shape
    out = np.empty((B, H, hd), dtype=np.int64)
    for b in range(B):
        out[b] = attention_cached(q[b][:, None, :], ks[b], vs[b], ks[b].shape[1] - 1, frac, inv_sqrt)[:, 0, :]
    return out


def producer_overflow(qh: np.ndarray, k: np.ndarray, v: np.ndarray, start: int, frac: int, inv_sqrt: int) -> bool:
    """True where a native producer returns rc 2: per (h, m), max|q_row|*max|K| > INT64_MAX/hd, or
    max|p_row|*max|V| > INT64_MAX/Lv with Lv = start+m+1 (bonsai_q1_kernel.c:1466-1500)."""
    H, M, hd = qh.shape
    Hkv, L, _ = k.shape
    rep = H // Hkv
    maxk = [fx.absmax(k[j]) for j in range(Hkv)]
    maxv = [fx.absmax(v[j]) for j in range(Hkv)]
    for h in range(H):
        kv = h // rep
        for m in range(M):
            if fx.absmax(qh[h, m]) * maxk[kv] > fx.INT64_MAX // hd:
                return True
    # probs are <= 2^frac; check the PV bound with the exact probs
    with np.errstate(over="ignore"):
        for h in range(H):
            kv = h // rep
            for m in range(M):
                lv = start + m + 1
                s = (qh[h, m] @ k[kv, :lv].T) >> np.int64(frac)
                s = (s * np.int64(inv_sqrt)) >> np.int64(frac)
                p = fx.softmax_rows(s[None], frac)[0]
                if fx.absmax(p) * maxv[kv] > fx.INT64_MAX // lv:
                    return True
    return False
