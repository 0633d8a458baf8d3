"""Seeded synthetic workloads for the BASELINE configs (test infrastructure).

Every tensor is drawn from ``oracle.prng`` keyed by (seed, tensor id), so the GPU tests regenerate bit-identical
inputs anywhere. Distributions follow the survey's measurement plan: Q1 bits uniform, scales U[1, 2^12] (the real
model has small positive scales), gains U[2^15, 2^17], residual inputs U[-2^20, 2^20], KV U[-2^20, 2^20).
"""
from __future__ import annotations

import numpy as np

from . import prng
from .rope import bonsai8b_tables, build_rope_tables

PROJ = ("wq", "wk", "wv", "wo", "w1", "wu", "w2")


def q1_weight(seed: int, tid: int, out_f: int, in_f: int, smin: int = 1, smax: int = 1 << 12):
    nb = in_f // 128
    bits = prng.uniform_bytes(seed, tid, (out_f, nb, 16))
    scale = prng.uniform_int(seed, tid + 1, (out_f, nb), smin, smax + 1)
    return bits, scale


def bonsai_layer(seed: int, d: int, H: int, Hkv: int, hd: int, dff: int, li: int = 0) -> dict:
    base = 1000 * (li + 1)
    shapes = {"wq": (H * hd, d), "wk": (Hkv * hd, d), "wv": (Hkv * hd, d), "wo": (d, H * hd),
              "w1": (dff, d), "wu": (dff, d), "w2": (d, dff)}
    layer = {}
    for i, name in enumerate(PROJ):
        layer[name] = q1_weight(seed, base + 10 * i, *shapes[name])
    layer["n1g"] = prng.uniform_int(seed, base + 100, (d,), 1 << 15, (1 << 17) + 1)
    layer["n2g"] = prng.uniform_int(seed, base + 101, (d,), 1 << 15, (1 << 17) + 1)
    layer["qng"] = prng.uniform_int(seed, base + 102, (hd,), 1 << 15, (1 << 17) + 1)
    layer["kng"] = prng.uniform_int(seed, base + 103, (hd,), 1 << 15, (1 << 17) + 1)
    return layer


def bonsai_model(seed: int, *, d: int, H: int, Hkv: int, hd: int, dff: int, n_layers: int, vocab: int,
                 ctx: int, yarn: bool = False) -> dict:
    cfg = {"d": d, "H": H, "Hkv": Hkv, "hd": hd, "dff": dff, "n_layers": n_layers, "vocab": vocab, "frac": 16}
    layers = [bonsai_layer(seed, d, H, Hkv, hd, dff, li) for li in range(n_layers)]
    cos, sin = bonsai8b_tables(ctx) if yarn else build_rope_tables(ctx, hd, 1_000_000, 16)
    return {
        "cfg": cfg, "layers": layers, "cos": cos, "sin": sin,
        "embed": q1_weight(seed, 7, vocab, d), "out": q1_weight(seed, 9, vocab, d),
        "final_g": prng.uniform_int(seed, 11, (d,), 1 << 15, (1 << 17) + 1),
    }


def small_bonsai(seed: int = 0, *, ctx: int = 64) -> dict:
    """2-layer d=128, H=4/2, hd=32, dff=256, vocab=256 (the reference's smoke-test shape,
    bonsai/tests/test_bonsai_smoke.py:26-32) with our seeded draws."""
    return bonsai_model(seed, d=128, H=4, Hkv=2, hd=32, dff=256, n_layers=2, vocab=256, ctx=ctx)


def kv_fill(seed: int, tid: int, Hkv: int, L: int, hd: int, mag: int = 1 << 20):
    k = prng.uniform_int(seed, tid, (Hkv, L, hd), -mag, mag)
    v = prng.uniform_int(seed, tid + 1, (Hkv, L, hd), -mag, mag)
    return k, v


def kv_fill_seq(seed: int, layer: int, kind: int, sid: int, Hkv: int, L: int, hd: int, lo: int = -(1 << 20),
                hi: int = 1 << 20):
    """The device cache generator's draw (kv_fill_kernel): (Hkv, L, hd) for one layer, kind (0 K, 1 V), sequence
    id."""
    return prng.uniform_int(seed, 100000 + 1024 * layer + 512 * kind + sid, (Hkv, L, hd), lo, hi)
