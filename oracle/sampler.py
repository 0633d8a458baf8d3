"""The reference engine's integer samplers, restated in numpy + hashlib (test infrastructure only).

Restates ``bonsai/src/trinote/infer_int/sampler.py``:

* ``apply_rep_penalty`` (:182-211): CTRL penalty ``l*FP // (FP+p)`` (l >= 0) / ``l*(FP+p) // FP`` (l < 0) on every
  token seen in the history, then the no-repeat-n-gram ban to ``-(1 << 40)`` (:176);
* ``_apply_temp_fp`` (:261-275): ``(logit * inv_temp_fp) >> frac`` with the fail-loud int64 guard on the peak
  magnitude;
* ``_probs_fp`` (:318-323): the engine's fixed-point softmax over the (temperature-scaled) row;
* ``_truncate`` (:351-381): top-k / nucleus over the stable descending order (ties: higher token id first),
  always keeping one token;
* ``_truncate_min_p`` (:384-400);
* ``_prng_word`` / ``draw_uniform_int`` (:283-315): the SHA-256 counter word keyed by (seed, position, counter),
  reduced to ``[0, total)`` by Lemire's multiply-shift with rejection;
* ``sample_token`` (:403-437).

Pinned by (tests/test_oracle_sampler.py): the truncation known answers of
``bonsai/tests/test_sampler_truncation.py:55-94`` (high-id tie at the top-k boundary, nucleus crossing, all-zero
fallback) and its stable-sort property oracle (:9-52) on the same tiny tie-heavy rows; SHA-256 against the FIPS
180-2 "abc" vector (through hashlib, the same primitive); Lemire's reduction against the closed form
``floor(x * n / 2^64)`` and its rejection threshold ``2^64 mod n`` on brute-forced small cases; the repetition
penalty against Python big-int floor division; and greedy == numpy first-max.
"""
from __future__ import annotations

import hashlib

import numpy as np

from .fixedpoint import softmax_rows

MODES = {"greedy": 0, "temp": 1, "top_k": 2, "top_p": 3, "min_p": 4}
NGRAM_BAN = -(1 << 40)
PRNG_TAG = b"trinote-sampler-draw/v1"
MASK64 = (1 << 64) - 1


def apply_rep_penalty(row: np.ndarray, hist, rep_penalty_fp: int, no_repeat_ngram: int, frac: int) -> np.ndarray:
    row = np.array(row, dtype=np.int64)
    hist = [int(x) for x in hist]
    if not hist:
        return row
    if rep_penalty_fp:
        fp = 1 << frac
        den = fp + int(rep_penalty_fp)
        for t in set(hist):
            v = int(row[t])
            # numpy int64 products wrap mod 2^64 before the floor division (sampler.py:203)
            prod = (v * fp) if v >= 0 else (v * den)
            prod = ((prod + (1 << 63)) & MASK64) - (1 << 63)
            row[t] = prod // den if v >= 0 else prod // fp
    n = int(no_repeat_ngram)
    if n > 1 and len(hist) >= n:
        prefix = tuple(hist[-(n - 1):])
        for i in range(len(hist) - n + 1):
            if tuple(hist[i:i + n - 1]) == prefix:
                row[hist[i + n - 1]] = NGRAM_BAN
    return row


def apply_temp(row: np.ndarray, inv_temp: int, frac: int) -> np.ndarray:
    """Raises OverflowError where the reference does (peak * inv_temp >= 2^63)."""
    row = np.asarray(row, dtype=np.int64)
    lo, hi = int(row.min(initial=0)), int(row.max(initial=0))
    if max(abs(lo), abs(hi)) * int(inv_temp) >= (1 << 63):
        raise OverflowError("temperature scaling overflows int64")
    return (row * np.int64(inv_temp)) >> np.int64(frac)


def probs(row: np.ndarray, inv_temp: int, frac: int) -> np.ndarray:
    row = np.asarray(row, dtype=np.int64)
    if inv_temp != (1 << frac):
        row = apply_temp(row, inv_temp, frac)
    return softmax_rows(row[None, :], frac)[0]


def truncate(p: np.ndarray, top_k: int, top_p_fp: int, frac: int) -> np.ndarray:
    p = np.asarray(p, dtype=np.int64)
    count = int(p.shape[0])
    order = np.argsort(p, kind="stable")[::-1]
    keep = min(max(1, top_k), count) if top_k and top_k > 0 else count
    if top_p_fp < (1 << frac):
        csum = np.cumsum(p[order[:keep]])
        n = int(np.searchsorted(csum, int(top_p_fp), side="left")) + 1
        keep = max(1, min(n, keep))
    out = np.zeros_like(p)
    kept = order[:keep]
    out[kept] = p[kept]
    if not out.any():
        out[int(order[0])] = 1
    return out


def truncate_min_p(p: np.ndarray, min_p_fp: int, frac: int) -> np.ndarray:
    p = np.asarray(p, dtype=np.int64).copy()
    if min_p_fp <= 0:
        return p
    amax = int(p.argmax())
    pmax = int(p[amax])
    if pmax <= 0:
        return p
    thresh = (int(min_p_fp) * pmax) >> frac
    p[p < np.int64(thresh)] = 0
    if not p.any():
        p[amax] = 1
    return p


def prng_word(seed: int, position: int, counter: int) -> int:
    msg = (PRNG_TAG + (seed & MASK64).to_bytes(8, "big") + (position & MASK64).to_bytes(8, "big")
           + (counter & MASK64).to_bytes(8, "big"))
    return int.from_bytes(hashlib.sha256(msg).digest()[:8], "big")


def draw_uniform_int(total: int, seed: int, position: int) -> int:
    n = int(total)
    if n <= 1:
        return 0
    j = 0
    m = prng_word(seed, position, j) * n
    j += 1
    low = m & MASK64
    if low < n:
        t = (1 << 64) % n
        while low < t:
            m = prng_word(seed, position, j) * n
            j += 1
            low = m & MASK64
    return m >> 64


def sample_token(row: np.ndarray, mode: str, frac: int, *, inv_temp: int | None = None, top_k: int = 0,
                 top_p_fp: int | None = None, min_p_fp: int = 0, seed: int = 0, position: int = 0,
                 hist=None, rep_penalty: int = 0, no_repeat_ngram: int = 0) -> int:
    """sample_token with the committed fixed-point settings (inv_temp / top_p_fp default to the identities)."""
    inv_temp = (1 << frac) if inv_temp is None else int(inv_temp)
    top_p_fp = (1 << frac) if top_p_fp is None else int(top_p_fp)
    if (rep_penalty or no_repeat_ngram) and hist is not None:
        row = apply_rep_penalty(row, hist, rep_penalty, no_repeat_ngram, frac)
    row = np.asarray(row, dtype=np.int64)
    if mode == "greedy":
        return int(row.argmax())
    p = probs(row, inv_temp, frac)
    if mode in ("top_k", "top_p"):
        p = truncate(p, top_k, top_p_fp, frac)
    elif mode == "min_p":
        p = truncate_min_p(p, min_p_fp, frac)
    total = int(p.sum())
    if total <= 0:
        return int(row.argmax())
    target = draw_uniform_int(total, seed, position)
    return int(np.searchsorted(np.cumsum(p), target, side="right"))
