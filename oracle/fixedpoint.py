"""Fixed-point primitives of the reference engine, restated in numpy (test infrastructure).

Restates ``bonsai/src/trinote/determinism/fixedpoint.py`` (RMSNorm :31-71, ``_exp2_neg_fixed`` :74-96, softmax
:99-140, sigmoid :143-174, ``_scaled_log2e`` :177-179, guarded matmul :207-240) and the SiLU wrapper
``reference_bonsai.fixed_point_silu`` (:245-264). numpy int64 semantics are the contract: ``*``/``+`` wrap mod
2^64, ``>>`` is an arithmetic (floor) shift whose out-of-range counts (negative or >= 64) give 0 / -1, ``//``
floors.

Pinned by (tests/test_oracle_core.py): the sigmoid == softmax([0, x])[1] identity
(``bonsai/tests/test_bonsai_smoke.py:468-484``); exp2 closed-form values at integer exponents (2^-k exactly);
RMSNorm against Python ``math.isqrt`` + big-int floor division on random rows and against the compiled
reference C kernel (``oracle/_ref``) where present; SiLU / attention against the compiled reference C kernel at
int64 extremes.
"""
from __future__ import annotations

import math

import numpy as np

LOG2E_Q16 = 94548
C0, C1, C2, C3 = 65536, 45426, 15743, 3638
NEG_INF_SHIFT = 30
INT64_MAX = (1 << 63) - 1


def scaled_log2e(frac: int) -> int:
    shift = 16 - frac
    return LOG2E_Q16 >> shift if shift >= 0 else LOG2E_Q16 << (-shift)


def d_clip(frac: int, *, hard_cap: bool = True) -> int:
    """Distance past which 2^-d floors to 0 (fixedpoint.py:120). nmc's vendored copy has no hard cap
    (north-mini-code/src/nmc/_bonsai/fixedpoint.py:148); the two agree for frac <= 28."""
    log2e = scaled_log2e(frac)
    first = ((frac + 2) << (2 * frac)) // log2e
    return min(first, (1 << 62) // log2e) if hard_cap else first


def rshift(a: np.ndarray, s) -> np.ndarray:
    """numpy's int64 ``a >> s`` with explicit out-of-range behaviour (count < 0 or >= 64 -> 0 / -1)."""
    a = np.asarray(a, dtype=np.int64)
    s = np.asarray(s, dtype=np.int64)
    ok = (s >= 0) & (s < 64)
    sc = np.where(ok, s, 0)
    return np.where(ok, a >> sc, np.where(a < 0, np.int64(-1), np.int64(0)))


def exp2_neg_fixed(u: np.ndarray, frac: int) -> np.ndarray:
    """2^-(u / 2^frac) as a cubic polynomial on the fraction and a shift by the integer part (fixedpoint.py:74)."""
    u = np.asarray(u, dtype=np.int64)
    fp = np.int64(1 << frac)
    k = u >> np.int64(frac)
    f = u & (fp - 1)
    shift = 16 - frac
    if shift >= 0:
        c0, c1, c2, c3 = (C0 >> shift, C1 >> shift, C2 >> shift, C3 >> shift)
    else:
        c0, c1, c2, c3 = (C0 << -shift, C1 << -shift, C2 << -shift, C3 << -shift)
    with np.errstate(over="ignore"):
        f2 = (f * f) >> np.int64(frac)
        f3 = (f2 * f) >> np.int64(frac)
        poly = (np.int64(c0) - ((np.int64(c1) * f) >> np.int64(frac)) + ((np.int64(c2) * f2) >> np.int64(frac))
                - ((np.int64(c3) * f3) >> np.int64(frac)))
    poly = np.maximum(poly, 0)
    kk = np.minimum(k, 63)
    return rshift(poly, kk)


def softmax_rows(z: np.ndarray, frac: int) -> np.ndarray:
    """Row-wise fixed-point softmax (fixedpoint.py:99-140)."""
    assert 1 <= frac <= 29
    z = np.atleast_2d(np.asarray(z, dtype=np.int64))
    log2e = np.int64(scaled_log2e(frac))
    dc = np.int64(d_clip(frac))
    out = np.empty(z.shape, dtype=np.int64)
    with np.errstate(over="ignore"):
        for r in range(z.shape[0]):
            row = z[r]
            m = row.max()
            d = np.minimum(m - row, dc)
            u = (d * log2e) >> np.int64(frac)
            e = exp2_neg_fixed(u, frac)
            zsum = int(e.sum())
            out[r] = 0 if zsum == 0 else (e << np.int64(frac)) // np.int64(zsum)
    return out


def sigmoid(x: np.ndarray, frac: int, *, hard_cap: bool = True) -> np.ndarray:
    """Fixed-point sigmoid == softmax([0, x])[1] (fixedpoint.py:143-174)."""
    assert 1 <= frac <= 29
    x = np.asarray(x, dtype=np.int64)
    log2e = np.int64(scaled_log2e(frac))
    dc = np.int64(d_clip(frac, hard_cap=hard_cap))
    with np.errstate(over="ignore"):
        m = np.maximum(x, 0)
        d0 = np.minimum(m, dc)
        d1 = np.minimum(m - x, dc)
        e0 = exp2_neg_fixed((d0 * log2e) >> np.int64(frac), frac)
        e1 = exp2_neg_fixed((d1 * log2e) >> np.int64(frac), frac)
        z = e0 + e1
        out = np.zeros(x.shape, dtype=np.int64)
        np.floor_divide(e1 << np.int64(frac), z, out=out, where=(z != 0), casting="unsafe")
    return out


def silu_wrap(x: np.ndarray, frac: int) -> np.ndarray:
    """Bonsai SiLU ``(x * sigmoid(x)) >> frac`` wrapping mod 2^64 (reference_bonsai.py:245-264)."""
    x = np.asarray(x, dtype=np.int64)
    with np.errstate(over="ignore"):
        return (x * sigmoid(x, frac)) >> np.int64(frac)


def mulshift_wrap(a: np.ndarray, b: np.ndarray, frac: int) -> np.ndarray:
    """``(a * b) >> frac`` in int64 with wrap (reference_bonsai.py:614)."""
    with np.errstate(over="ignore"):
        return (np.asarray(a, np.int64) * np.asarray(b, np.int64)) >> np.int64(frac)


def add_wrap(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return np.asarray(a, np.int64) + np.asarray(b, np.int64)


def absmax(a: np.ndarray) -> int:
    a = np.asarray(a)
    return max(abs(int(a.min())), abs(int(a.max()))) if a.size else 0


def assert_no_int64_overflow(a: np.ndarray, b: np.ndarray) -> None:
    """max|a| * max|b| * K must fit int64 (fixedpoint.py:207-227); raises OverflowError otherwise."""
    if a.size == 0 or b.size == 0:
        return
    k = a.shape[-1]
    bound = absmax(a) * absmax(b) * int(k)
    if bound > INT64_MAX:
        raise OverflowError(f"fixed_point_matmul bound {bound} > 2^63-1 (K={k})")


def fixed_point_matmul(a: np.ndarray, b: np.ndarray, frac: int) -> np.ndarray:
    """``(A @ B) >> frac`` with the fail-loud int64 bound (fixedpoint.py:230-240)."""
    a = np.asarray(a, dtype=np.int64)
    b = np.asarray(b, dtype=np.int64)
    assert_no_int64_overflow(a, b)
    return (a @ b) >> np.int64(frac)


def rmsnorm(x: np.ndarray, frac: int, eps: int = 1, gain: np.ndarray | None = None) -> np.ndarray:
    """Integer RMSNorm (fixedpoint.py:31-71): exact ssq, isqrt, floor division, int64 gain with envelope raise."""
    x = np.atleast_2d(np.asarray(x, dtype=np.int64))
    rows, n = x.shape
    out = np.empty(x.shape, dtype=np.int64)
    mx = absmax(x)
    small = mx * mx * n <= INT64_MAX and mx < (1 << (62 - frac))
    if small:
        ssq = (x * x).sum(axis=1)
        for r in range(rows):
            rms = math.isqrt(int(ssq[r]) // n + eps)
            out[r] = (x[r] << np.int64(frac)) // np.int64(rms)
    else:
        for r in range(rows):
            rowo = x[r].astype(object)
            ssq = int(np.dot(rowo, rowo))
            rms = math.isqrt(ssq // n + eps)
            out[r] = ((rowo << frac) // rms).astype(np.int64)
    if gain is not None:
        g = np.asarray(gain, dtype=np.int64)
        if out.size and g.size and absmax(out) * absmax(g) > INT64_MAX:
            raise OverflowError("rmsnorm gain multiply would overflow int64")
        out = (out * g) >> np.int64(frac)
    return out


def inv_sqrt_fp(head_dim: int, frac: int) -> int:
    """``round((1/sqrt(hd)) * 2^frac)`` (reference_bonsai.py:563); 5793 at hd=128, frac=16."""
    return int(round((1.0 / np.sqrt(head_dim)) * (1 << frac)))
