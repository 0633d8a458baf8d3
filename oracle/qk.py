"""north-mini-code Q4_K / Q6_K integer codec, exact linear and the MoE block, restated (test infrastructure).

Follows ``north-mini-code/src/nmc/qk_codec.py`` (``get_scale_min_k4`` :28-35, ``dequant_q4k_int`` :54-71,
``dequant_q6k_int`` :114-131, whole-tensor forms :158-206), ``cohere2.py`` (``linear`` :102-106, ``silu_int``
:109-111, ``_topk_lowidx`` :162-165, ``moe_layer_int`` :168-188) and the vendored sigmoid without the hard cap
(``north-mini-code/src/nmc/_bonsai/fixedpoint.py:148``).

The fp16 -> fixed conversion ``round(float(fp16) * 2^fw)`` is restated in integers from the fp16 bits.

Pinned by: the compiled reference CPU kernel ``qk_linear`` (oracle/_ref, from nmc_qk_kernel.c) on random
blocks; the reference's scalar per-block codec rule restated per element (tests/test_oracle_qk.py) and a
hand-built block whose dequantized weights are known in closed form; ``fp16_fixed`` against Python's
``round(float(np.float16)...)`` over every finite fp16 bit pattern.
"""
from __future__ import annotations

import numpy as np

from . import fixedpoint as fx
from . import prng

QK_K = 256
BS = {0: 144, 1: 210}


def fp16_fixed(h: np.ndarray, fw: int) -> np.ndarray:
    """round_half_even(fp16(h) * 2^fw) as int64, computed from the bit patterns (vectorised)."""
    h = np.asarray(h, dtype=np.int64) & 0xFFFF
    sign = (h >> 15) & 1
    e = (h >> 10) & 31
    mant = h & 0x3FF
    m = np.where(e == 0, mant, mant | 0x400)
    sh = np.where(e == 0, fw - 24, e - 25 + fw)
    out = np.zeros(h.shape, dtype=object)
    for idx in np.ndindex(h.shape):
        mm, s = int(m[idx]), int(sh[idx])
        if s >= 0:
            r = mm << s
        else:
            q, rem = mm >> -s, mm & ((1 << -s) - 1)
            half = 1 << (-s - 1)
            r = q + (1 if (rem > half or (rem == half and (q & 1))) else 0)
        out[idx] = -r if sign[idx] else r
    return out.astype(np.int64)


def _scale_min(scales: np.ndarray):
    """(nb, 12) packed -> sc, m (nb, 8) per get_scale_min_k4."""
    s = scales.astype(np.int64)
    sc = np.empty((s.shape[0], 8), np.int64)
    mn = np.empty((s.shape[0], 8), np.int64)
    for j in range(8):
        if j < 4:
            sc[:, j] = s[:, j] & 63
            mn[:, j] = s[:, j + 4] & 63
        else:
            sc[:, j] = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
            mn[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    return sc, mn


def dequant(raw: np.ndarray, out_f: int, nb: int, qtype: int, fw: int) -> np.ndarray:
    """Raw block bytes (out_f * nb blocks, row-major) -> W (out_f, nb*256) int64 at scale 2^fw."""
    b = np.asarray(raw, dtype=np.uint8).reshape(out_f * nb, BS[qtype])
    n = b.shape[0]
    if qtype == 0:
        dq = fp16_fixed(b[:, 0].astype(np.int64) | (b[:, 1].astype(np.int64) << 8), fw)[:, None]
        dmq = fp16_fixed(b[:, 2].astype(np.int64) | (b[:, 3].astype(np.int64) << 8), fw)[:, None]
        sc, mn = _scale_min(b[:, 4:16])
        qs = b[:, 16:144].astype(np.int64)
        w = np.empty((n, QK_K), np.int64)
        for g in range(4):
            lo = qs[:, 32 * g:32 * g + 32] & 0xF
            hi = qs[:, 32 * g:32 * g + 32] >> 4
            w[:, 64 * g:64 * g + 32] = dq * sc[:, 2 * g:2 * g + 1] * lo - dmq * mn[:, 2 * g:2 * g + 1]
            w[:, 64 * g + 32:64 * g + 64] = dq * sc[:, 2 * g + 1:2 * g + 2] * hi - dmq * mn[:, 2 * g + 1:2 * g + 2]
    else:
        ql = b[:, 0:128].astype(np.int64)
        qh = b[:, 128:192].astype(np.int64)
        sca = b[:, 192:208].view(np.int8).astype(np.int64)
        dq = fp16_fixed(b[:, 208].astype(np.int64) | (b[:, 209].astype(np.int64) << 8), fw)[:, None]
        w = np.empty((n, QK_K), np.int64)
        l = np.arange(32)
        is_ = l // 16
        for half in range(2):
            qlo, qho, sco, yo = 64 * half, 32 * half, 8 * half, 128 * half
            Ql, Ql2, Qh = ql[:, qlo:qlo + 32], ql[:, qlo + 32:qlo + 64], qh[:, qho:qho + 32]
            qq = [((Ql & 0xF) | (((Qh >> 0) & 3) << 4)) - 32, ((Ql2 & 0xF) | (((Qh >> 2) & 3) << 4)) - 32,
                  ((Ql >> 4) | (((Qh >> 4) & 3) << 4)) - 32, ((Ql2 >> 4) | (((Qh >> 6) & 3) << 4)) - 32]
            for k in range(4):
                w[:, yo + 32 * k:yo + 32 * k + 32] = dq * sca[:, sco + is_ + 2 * k] * qq[k]
    return w.reshape(out_f, nb * QK_K)


def linear(x: np.ndarray, W: np.ndarray, fw: int) -> np.ndarray:
    """Exact ``(x @ W.T) >> fw`` in Python big-ints, then int64 (raises like cohere2.linear)."""
    xo = np.atleast_2d(np.asarray(x, dtype=np.int64)).astype(object)
    return ((xo @ np.asarray(W, dtype=np.int64).astype(object).T) >> fw).astype(np.int64)


def silu_int(x: np.ndarray, fa: int) -> np.ndarray:
    sig = fx.sigmoid(np.asarray(x, np.int64), fa, hard_cap=False)
    return ((np.asarray(x, object) * np.asarray(sig, object)) >> fa).astype(np.int64)


def topk_lowidx(logits_row: np.ndarray, k: int) -> np.ndarray:
    return np.argsort(-np.asarray(logits_row, dtype=np.int64), kind="stable")[:k]


def moe_route(router_logits: np.ndarray, k: int, fa: int):
    """(sel (m, k) expert ids, gates (m, k)) from router logits: stable top-k + sigmoid gates."""
    sel = np.stack([topk_lowidx(r, k) for r in router_logits])
    gates = np.stack([fx.sigmoid(r[s].astype(np.int64), fa, hard_cap=False) for r, s in zip(router_logits, sel)])
    return sel, gates


def moe_ffn(h: np.ndarray, sel: np.ndarray, gates: np.ndarray, experts: dict, fa: int, fw: int, lin=None) -> np.ndarray:
    """cohere2.moe_layer_int after routing: out[t] = sum_j (down_e(silu(gate_e h) * up_e h >> fa) * g_j) >> fa.
    ``experts[e]`` = dict(gate=Wg, up=Wu, down=Wd) dequantized int64 matrices; ``lin`` overrides the exact linear
    (e.g. the C restatement) with the same signature."""
    lin = lin or linear
    m, d = h.shape
    out = np.zeros((m, d), dtype=object)
    for t in range(m):
        ht = h[t:t + 1]
        for j, e in enumerate(sel[t]):
            ex = experts[int(e)]
            g = silu_int(lin(ht, ex["gate"], fw), fa)
            u = lin(ht, ex["up"], fw)
            gu = ((g.astype(object) * u.astype(object)) >> fa).astype(np.int64)
            eo = lin(gu, ex["down"], fw)[0].astype(object)
            out[t] += (eo * int(gates[t, j])) >> fa
    return out.astype(np.int64)


def moe_ffn_grouped(h: np.ndarray, sel: np.ndarray, gates: np.ndarray, experts: dict, fa: int, fw: int,
                    lin) -> np.ndarray:
    """Same value as ``moe_ffn``, evaluated expert by expert: the (token, slot) pairs routed to one expert share
    its gate/up/down linears (each pair's arithmetic is unchanged; the per-token combine is an exact big-int sum,
    so the order of the terms does not matter). ``lin(x, experts[e][name], fw)`` evaluates one exact linear."""
    m, d = h.shape
    out = np.zeros((m, d), dtype=object)
    pairs: dict = {}
    for t in range(m):
        for j, e in enumerate(sel[t]):
            pairs.setdefault(int(e), []).append((t, j))
    for e, lst in pairs.items():
        rows = np.array([t for t, _ in lst])
        g = silu_int(lin(h[rows], experts[e]["gate"], fw), fa)
        u = lin(h[rows], experts[e]["up"], fw)
        gu = ((g.astype(object) * u.astype(object)) >> fa).astype(np.int64)
        dn = lin(gu, experts[e]["down"], fw)
        for i, (t, j) in enumerate(lst):
            out[t] += (dn[i].astype(object) * int(gates[t, j])) >> fa
    return out.astype(np.int64)


def random_blocks(seed: int, tid: int, out_f: int, nb: int, qtype: int, *, dlo=0.002, dhi=0.01, dminhi=0.005):
    """Seeded raw blocks: fp16 d ~ U[dlo, dhi], dmin ~ U[0, dminhi] (Q4_K), random scale / quant bytes."""
    n = out_f * nb
    raw = prng.uniform_bytes(seed, tid, (n, BS[qtype]))
    u = prng.stream(seed, tid + 1, 2 * n).astype(np.float64) / 2.0 ** 64
    d = (dlo + (dhi - dlo) * u[:n]).astype(np.float16).view(np.uint16)
    if qtype == 0:
        dmin = (dminhi * u[n:]).astype(np.float16).view(np.uint16)
        raw[:, 0] = d & 0xFF
        raw[:, 1] = d >> 8
        raw[:, 2] = dmin & 0xFF
        raw[:, 3] = dmin >> 8
    else:
        raw[:, 208] = d & 0xFF
        raw[:, 209] = d >> 8
    return raw.reshape(-1)
