"""Packed Q1_0 linear, restated (test infrastructure).

Follows ``bonsai/src/trinote/infer_int/reference_bonsai.py:149-219`` (``q1_linear_ref``), ``:131-135``
(``_unpack_q1_signs``: bit i of byte j is weight 8j+i, little-endian, 1 -> +1, 0 -> -1), ``:138-146``
(``q1_rows_fp``) and the lowest-index argmax of ``:812-827``:

    out[t, o] = sum_b ( (sum_{i in block b} sign[o, i] * x[t, i]) * scale[o, b] ) >> frac      (mod 2^64)

Pinned by (tests/test_oracle_core.py): Python big-int brute force reduced mod 2^64 on small shapes (incl. int64
extrema and frac in {0, 1, 16, 31, 62}); the hand-derived wrap KAT of ``bonsai/tests/test_bonsai_smoke.py:890-906``
(x=2^62, frac=1, scales 3/-3/4 -> [-2^61, 2^61, 0]); the ``2*pos - total`` identity; and the compiled reference C
kernel ``bonsai_q1_linear_i64`` (``oracle/_ref``) where present.
"""
from __future__ import annotations

import numpy as np

GROUP = 128
MASK64 = (1 << 64) - 1


def unpack_signs(bits: np.ndarray) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint8)
    u = np.unpackbits(b, axis=-1, bitorder="little").astype(np.int8)
    return (u * 2 - 1).astype(np.int8)


def q1_linear(x: np.ndarray, bits: np.ndarray, scale: np.ndarray, frac: int, *, chunk: int = 512) -> np.ndarray:
    """Expanded-sign form of the Q1_0 linear in int64 numpy (wraps mod 2^64 like the reference)."""
    x = np.atleast_2d(np.asarray(x, dtype=np.int64))
    s = np.asarray(scale, dtype=np.int64)
    n_out, nb = s.shape
    if x.shape[1] != nb * GROUP:
        raise ValueError("Q1_0 contraction mismatch")
    xg = x.reshape(x.shape[0], nb, GROUP)
    out = np.empty((x.shape[0], n_out), dtype=np.int64)
    with np.errstate(over="ignore"):
        for lo in range(0, n_out, chunk):
            hi = min(lo + chunk, n_out)
            signs = unpack_signs(bits[lo:hi]).astype(np.int64)
            acc = np.einsum("tbi,obi->tob", xg, signs)
            out[:, lo:hi] = ((acc * s[lo:hi][None]) >> np.int64(frac)).sum(axis=2, dtype=np.int64)
    return out


def q1_linear_bigint(x, bits, scale, frac: int) -> np.ndarray:
    """Brute-force Python big-int restatement, each step reduced mod 2^64 (tiny shapes only)."""
    x = np.atleast_2d(np.asarray(x, dtype=np.int64))
    s = np.asarray(scale, dtype=np.int64)
    signs = unpack_signs(bits)
    n_out, nb = s.shape

    def to_signed(v):
        v &= MASK64
        return v - (1 << 64) if v >> 63 else v

    out = np.empty((x.shape[0], n_out), dtype=np.int64)
    for t in range(x.shape[0]):
        for o in range(n_out):
            tot = 0
            for b in range(nb):
                acc = sum(int(signs[o, b, i]) * int(x[t, b * GROUP + i]) for i in range(GROUP))
                prod = to_signed(to_signed(acc) * int(s[o, b]))
                tot += prod >> frac if frac < 64 else (-1 if prod < 0 else 0)
            out[t, o] = to_signed(tot)
    return out


def q1_rows(bits, scale, rows) -> np.ndarray:
    """Embedding rows ``sign * scale`` (no frac shift), reference_bonsai.py:138-146."""
    idx = np.asarray(rows, dtype=np.int64)
    signs = unpack_signs(bits[idx]).astype(np.int64)
    sc = np.asarray(scale[idx], dtype=np.int64)
    return (signs * sc[:, :, None]).reshape(idx.shape[0], -1)


def argmax_lowest(logits: np.ndarray) -> np.ndarray:
    """Row argmax with the lowest index on ties (numpy first-max)."""
    return np.asarray(np.atleast_2d(logits).argmax(axis=1), dtype=np.int64)
