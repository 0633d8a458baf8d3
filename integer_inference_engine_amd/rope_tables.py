"""Fixed-point RoPE tables for the device path (built once on the host, then only read by the kernels).

Produces the int64 ``cos``/``sin`` tables of shape (positions, head_dim/2) at scale 2^frac that the reference
commits into its model artifact: plain RoPE (``bonsai/src/trinote/model/rope.py:42-66``) and llama.cpp-style
YaRN (``bonsai/src/trinote/model/rope_v2.py:43-89``). The per-element float expressions are evaluated in the
same IEEE order as the reference (the angle is advanced by repeated multiplication per pair index), with the
angle grid vectorised over positions and libm ``math.cos``/``math.sin`` per element, so the integers agree.
"""
from __future__ import annotations

import math

import numpy as np


def _quantise(theta: np.ndarray, mscale: float, scale: int):
    flat = theta.reshape(-1).tolist()
    c = np.fromiter((round(math.cos(t) * mscale * scale) for t in flat), dtype=np.int64, count=len(flat))
    s = np.fromiter((round(math.sin(t) * mscale * scale) for t in flat), dtype=np.int64, count=len(flat))
    return c.reshape(theta.shape), s.reshape(theta.shape)


def plain_tables(positions: int, head_dim: int, base: float = 10000, frac: int = 16):
    if head_dim % 2:
        raise ValueError("head_dim must be even")
    half = head_dim // 2
    inv = np.array([base ** (-(2 * i) / head_dim) for i in range(half)], dtype=np.float64)
    theta = np.arange(positions, dtype=np.float64)[:, None] * inv[None, :]
    return _quantise(theta, 1.0, 1 << frac)


def yarn_tables(positions: int, head_dim: int, *, base: float, freq_scale: float, n_ctx_orig: int,
                ext_factor: float = 1.0, attn_factor: float = 1.0, beta_fast: float = 32.0,
                beta_slow: float = 1.0, frac: int = 16):
    if head_dim % 2:
        raise ValueError("head_dim must be even")
    half = head_dim // 2
    base = float(base)

    def corr(beta):
        return head_dim * math.log(n_ctx_orig / (beta * 2 * math.pi)) / (2 * math.log(base))

    lo = max(0.0, float(math.floor(corr(beta_fast))))
    hi = min(float(head_dim - 1), float(math.ceil(corr(beta_slow))))
    step = base ** (-2.0 / head_dim)
    ms = attn_factor * ((1.0 + 0.1 * math.log(1.0 / freq_scale)) if ext_factor != 0.0 else 1.0)
    ext = np.empty((positions, half), dtype=np.float64)
    col = np.arange(positions, dtype=np.float64)
    for j in range(half):                   # theta_extrap(p, j) = ((p * step) * step) ... j times, as a loop
        ext[:, j] = col
        col = col * step
    theta = freq_scale * ext
    if ext_factor != 0.0:
        for j in range(half):
            y = (j - lo) / max(0.001, hi - lo)
            mix = (1.0 - min(1.0, max(0.0, y))) * ext_factor
            theta[:, j] = theta[:, j] * (1.0 - mix) + ext[:, j] * mix
    return _quantise(theta, ms, 1 << frac)


def bonsai8b_tables(positions: int):
    """Bonsai-8B (Qwen3-8B) YaRN tables: base 1e6, factor 4 (freq_scale 1/4), 16384 original context, hd 128."""
    return yarn_tables(positions, 128, base=1_000_000, freq_scale=0.25, n_ctx_orig=16_384)
