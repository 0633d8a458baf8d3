"""One M=1 decode step of a north-mini-code MoE block, restated (test infrastructure).

Follows ``north-mini-code/src/nmc/cohere2.py``: the parallel block ``x + Attn(n(x)) + MoE(n(x))`` (:191-199) with
one shared RMSNorm (:194), Q/K/V/O exact linears (:102-106), interleaved RoPE on sliding-window layers only
(:125-133, :197), GQA attention over the most recent ``window`` keys including the new one (:80-89, :136-161),
the router ``linear`` + lowest-index top-k + sigmoid gates and the SwiGLU experts (:162-188).

The decode step attends only the visible keys (the producer form); the full-sequence form in cohere2 adds
masked entries at ``-(1 << (fa + 30))``, which contribute exactly 0 unless every visible score lies below that
sentinel. The router's producer guard (nmc_qk_cuda.cu:615-638) refuses a row whose UNSHIFTED sum leaves int64;
``router_logits`` raises OverflowError there (the producer's rc 3).

Pinned by its parts: RMSNorm, softmax and sigmoid (oracle/fixedpoint.py), the exact Q4_K/Q6_K linear and the
MoE (oracle/qk.py), and the interleaved RoPE against the NeoX form on a permuted head (tests/test_oracle_qk.py);
and as a whole by tests/test_oracle_nmc_block.py: at every position of a sequence, for windows None / 1 / 3 /
S - 1 and with RoPE on sliding-window layers only, the decode step equals an independent full-sequence restatement
of cohere2's masked attention (:85-92, :136-161) and parallel block (:191-199).
"""
from __future__ import annotations

import numpy as np

from . import fixedpoint as fx
from . import qk
from .rope import apply_interleaved

INT64_MAX, INT64_MIN = (1 << 63) - 1, -(1 << 63)


def router_logits(h: np.ndarray, R: np.ndarray, fw: int) -> np.ndarray:
    """(h @ R.T) >> fw with exact sums; OverflowError where an unshifted sum leaves int64."""
    hs = np.atleast_2d(np.asarray(h, dtype=np.int64)).astype(object)
    acc = hs @ np.asarray(R, dtype=np.int64).astype(object).T
    for v in acc.ravel():
        if v > INT64_MAX or v < INT64_MIN:
            raise OverflowError("router sum leaves int64")
    return (acc >> fw).astype(np.int64)


def _narrow(v: int) -> int:
    if v > INT64_MAX or v < INT64_MIN:
        raise OverflowError("attention value leaves int64")
    return v


def attention_step(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, pos: int, window, fa: int, inv_sqrt: int) -> np.ndarray:
    """q (H, hd) of the new position `pos`; kc/vc (Hkv, >= pos+1, hd) including it. Returns (H, hd)."""
    H, hd = q.shape
    rep = H // kc.shape[0]
    first = pos - window + 1 if (window is not None and pos - window >= 0) else 0
    out = np.empty((H, hd), dtype=np.int64)
    for h in range(H):
        kv = h // rep
        scores = []
        for key in range(first, pos + 1):
            d = sum(int(a) * int(b) for a, b in zip(q[h], kc[kv, key]))
            scores.append(_narrow((_narrow(d >> fa) * inv_sqrt) >> fa))
        p = fx.softmax_rows(np.array(scores, dtype=np.int64)[None, :], fa)[0]
        for lane in range(hd):
            acc = sum(int(p[i]) * int(vc[kv, first + i, lane]) for i in range(len(p)))
            out[h, lane] = _narrow(acc >> fa)
    return out


def block_step(x: np.ndarray, W: dict, kc: np.ndarray, vc: np.ndarray, pos: int, window, rope: bool, cos, sin,
               cfg: dict, experts: dict):
    """x (1, d); W: dequantized int64 {wq, wk, wv, wo}, int64 gain (d,) and router (E, d); kc/vc (Hkv, cap, hd)
    with positions < pos filled. Returns (out (1, d), attention (1, d), ids, gates, new k row, new v row)."""
    fa, fw, H, Hkv, hd = cfg["fa"], cfg["fw"], cfg["H"], cfg["Hkv"], cfg["hd"]
    h = fx.rmsnorm(x, fa, cfg.get("eps", 1), W["gain"])
    q = qk.linear(h, W["wq"], fw).reshape(H, hd)
    k = qk.linear(h, W["wk"], fw).reshape(Hkv, hd)
    v = qk.linear(h, W["wv"], fw).reshape(Hkv, hd)
    if rope:
        q = apply_interleaved(q[:, None, :], cos[pos:pos + 1], sin[pos:pos + 1], fa)[:, 0, :]
        k = apply_interleaved(k[:, None, :], cos[pos:pos + 1], sin[pos:pos + 1], fa)[:, 0, :]
    kc, vc = kc.copy(), vc.copy()
    kc[:, pos], vc[:, pos] = k, v
    inv = fx.inv_sqrt_fp(hd, fa)
    att = attention_step(q, kc, vc, pos, window, fa, inv).reshape(1, H * hd)
    ao = qk.linear(att, W["wo"], fw)
    logits = router_logits(h, W["router"], fw)
    sel, gates = qk.moe_route(logits, cfg["used"], fa)
    moe = qk.moe_ffn(h, sel, gates, experts, fa, fw)
    with np.errstate(over="ignore"):
        out = np.asarray(x, np.int64) + ao + moe
    return out, ao, sel[0], gates[0], k, v
