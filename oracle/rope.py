"""RoPE tables and NeoX apply, restated (test infrastructure).

Table builders follow ``bonsai/src/trinote/model/rope.py:42-66`` (plain) and ``rope_v2.py:43-89`` (YaRN, the
llama.cpp ``rope_yarn`` blend). They call libm once at build time; the device path only reads the int64 table.
Apply follows ``rope_v2.py:92-117`` (rotate-half NeoX) with the overflow guard of ``rope.py:26-39``.

Pinned by the reference's KAT rows (``bonsai/tests/test_bonsai_smoke.py:91-107``) and by a committed sha256 of
the 8B-shape table (``tests/golden/rope_yarn_8b.json``) so the device table bytes are fixed.
"""
from __future__ import annotations

import hashlib
import math

import numpy as np

INT64_MAX = (1 << 63) - 1


def build_rope_tables(seq_len: int, head_dim: int, base: float = 10000, frac: int = 16):
    half = head_dim // 2
    scale = 1 << frac
    inv_freq = [base ** (-(2 * i) / head_dim) for i in range(half)]
    cos = np.empty((seq_len, half), dtype=np.int64)
    sin = np.empty((seq_len, half), dtype=np.int64)
    for p in range(seq_len):
        for i in range(half):
            ang = p * inv_freq[i]
            cos[p, i] = round(math.cos(ang) * scale)
            sin[p, i] = round(math.sin(ang) * scale)
    return cos, sin


def _corr_dim(n_dims, n_ctx_orig, n_rot, base):
    return n_dims * math.log(n_ctx_orig / (n_rot * 2 * math.pi)) / (2 * math.log(base))


def build_yarn_rope_tables(seq_len: int, head_dim: int, *, base: float, freq_scale: float, n_ctx_orig: int,
                           ext_factor: float = 1.0, attn_factor: float = 1.0, beta_fast: float = 32.0,
                           beta_slow: float = 1.0, frac: int = 16):
    half = head_dim // 2
    scale = 1 << frac
    lo = max(0.0, float(math.floor(_corr_dim(head_dim, n_ctx_orig, beta_fast, float(base)))))
    hi = min(float(head_dim - 1), float(math.ceil(_corr_dim(head_dim, n_ctx_orig, beta_slow, float(base)))))
    theta_scale = float(base) ** (-2.0 / head_dim)
    mscale_y = 1.0 + 0.1 * math.log(1.0 / freq_scale) if ext_factor != 0.0 else 1.0
    ramp = []
    for j in range(half):
        y = (j - lo) / max(0.001, hi - lo)          # i0 / 2 with i0 = 2j
        ramp.append((1.0 - min(1.0, max(0.0, y))) * ext_factor)
    cos = np.empty((seq_len, half), dtype=np.int64)
    sin = np.empty((seq_len, half), dtype=np.int64)
    for p in range(seq_len):
        theta_extrap = float(p)
        for j in range(half):
            theta = freq_scale * theta_extrap
            ms = attn_factor
            if ext_factor != 0.0:
                theta = theta * (1.0 - ramp[j]) + theta_extrap * ramp[j]
                ms *= mscale_y
            cos[p, j] = round(math.cos(theta) * ms * scale)
            sin[p, j] = round(math.sin(theta) * ms * scale)
            theta_extrap *= theta_scale
    return cos, sin


def bonsai8b_tables(seq_len: int):
    """Bonsai-8B YaRN tables (config_bonsai.py: base 1e6, factor 4, n_ctx_orig 16384, hd 128)."""
    return build_yarn_rope_tables(seq_len, 128, base=1_000_000, freq_scale=0.25, n_ctx_orig=16_384)


def table_hash(cos, sin) -> str:
    h = hashlib.sha256()
    h.update(np.ascontiguousarray(cos, dtype="<i8").tobytes())
    h.update(np.ascontiguousarray(sin, dtype="<i8").tobytes())
    return h.hexdigest()


def _absmax(a):
    return max(abs(int(a.min())), abs(int(a.max()))) if a.size else 0


def apply_neox(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, frac: int) -> np.ndarray:
    """x (..., seq, hd) rotated with rows cos[:seq] (rope_v2.py:92-117); raises on the int64 envelope."""
    x = np.asarray(x, dtype=np.int64)
    seq, hd = x.shape[-2], x.shape[-1]
    half = hd // 2
    c, s = cos[:seq], sin[:seq]
    if x.size and c.size and 2 * _absmax(x) * max(_absmax(c), _absmax(s)) > INT64_MAX:
        raise OverflowError("RoPE apply overflows int64")
    x0, x1 = x[..., :half], x[..., half:]
    out = np.empty_like(x)
    out[..., :half] = (x0 * c - x1 * s) >> np.int64(frac)
    out[..., half:] = (x0 * s + x1 * c) >> np.int64(frac)
    return out


def apply_neox_rows(x: np.ndarray, cos_rows: np.ndarray, sin_rows: np.ndarray, frac: int) -> np.ndarray:
    """Rotate x (B, n, hd) where row b uses its own table row (batched decode, reference_bonsai.py:745-756)."""
    x = np.asarray(x, dtype=np.int64)
    half = x.shape[-1] // 2
    c, s = cos_rows[:, None, :], sin_rows[:, None, :]
    out = np.empty_like(x)
    out[..., :half] = (x[..., :half] * c - x[..., half:] * s) >> np.int64(frac)
    out[..., half:] = (x[..., :half] * s + x[..., half:] * c) >> np.int64(frac)
    return out


def apply_interleaved(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, frac: int) -> np.ndarray:
    """Pairwise (x[2i], x[2i+1]) rotation of x (..., seq, hd) with rows cos[:seq] (the cohere2 / north-mini-code
    convention, north-mini-code/src/nmc/_bonsai/rope.py:79-100); raises on the int64 envelope (rope.py:26-39)."""
    x = np.asarray(x, dtype=np.int64)
    seq = x.shape[-2]
    c, s = cos[:seq], sin[:seq]
    if x.size and c.size and 2 * _absmax(x) * max(_absmax(c), _absmax(s)) > INT64_MAX:
        raise OverflowError("RoPE apply overflows int64")
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = (x0 * c - x1 * s) >> np.int64(frac)
    out[..., 1::2] = (x0 * s + x1 * c) >> np.int64(frac)
    return out
