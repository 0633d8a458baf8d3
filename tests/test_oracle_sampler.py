"""Pins the sampler oracle (oracle/sampler.py) before it checks the device sampler (CPU only).

Known answers come from the reference's own truncation tests (bonsai/tests/test_sampler_truncation.py); the other
checks use independent formulations: a boolean-mask stable-sort truncation, Python big-int floor division, the
closed form of Lemire's reduction, FIPS 180-2's SHA-256 vector, numpy's first-max."""
import hashlib

import numpy as np
import pytest

from oracle import sampler as smp
from oracle.fixedpoint import softmax_rows


def _mask_truncate(p, top_k, top_p_fp, frac):
    """Truncation by boolean masks over a stable ascending argsort reversed (an independent formulation)."""
    res = np.asarray(p, dtype=np.int64).copy()
    order = np.argsort(res, kind="stable")[::-1]
    keep = np.zeros(res.shape[0], dtype=bool)
    keep[order[: max(1, top_k)] if top_k and top_k > 0 else order] = True
    if top_p_fp < (1 << frac):
        running, n = 0, res.shape[0]
        for rank, i in enumerate(order):
            running += int(res[i])
            if running >= top_p_fp:
                n = rank + 1
                break
        nucleus = np.zeros(res.shape[0], dtype=bool)
        nucleus[order[: max(1, min(n, res.shape[0]))]] = True
        keep &= nucleus
    res[~keep] = 0
    if not res.any():
        res[int(order[0])] = 1
    return res


def test_truncate_known_answers():
    """bonsai/tests/test_sampler_truncation.py:55-94."""
    p = np.array([9, 10, 10, 10, 8, 10], dtype=np.int64)
    assert smp.truncate(p, 3, 1 << 16, 16).tolist() == [0, 0, 10, 10, 0, 10]      # high ids win the tie
    q = np.array([1, 2, 3, 5, 6, 7], dtype=np.int64)
    for tp, ids in ((7, [5]), (13, [4, 5]), (18, [3, 4, 5]), (100, [3, 4, 5])):
        assert np.flatnonzero(smp.truncate(q, 3, tp, 8)).tolist() == ids
    z = smp.truncate(np.zeros(32, dtype=np.int64), 7, 1, 16)
    assert z.tolist() == [0] * 31 + [1]


@pytest.mark.parametrize("size", [1, 2, 3, 7, 20, 21, 127, 257])
def test_truncate_matches_mask_formulation(size):
    """The tie-heavy sweep of test_sampler_truncation.py:30-52 against the boolean-mask formulation."""
    rng = np.random.default_rng(0xB035 + size)
    frac = 16
    rows = [np.zeros(size, dtype=np.int64), np.ones(size, dtype=np.int64), np.arange(size, dtype=np.int64) % 5]
    rows += [rng.integers(0, 33, size=size, dtype=np.int64) for _ in range(20)]
    for p in rows:
        for k in sorted({0, 1, 2, 3, 7, 20, max(1, size - 1), size, size + 3}):
            for tp in (0, 1, 7, 1 << 8, (1 << frac) - 1, 1 << frac):
                assert np.array_equal(smp.truncate(p, k, tp, frac), _mask_truncate(p, k, tp, frac))


def test_rep_penalty_and_ngram_against_bigint():
    rng = np.random.default_rng(3)
    frac, pen = 16, 13107
    row = rng.integers(-(1 << 40), 1 << 40, size=50, dtype=np.int64)
    hist = [3, 7, 3, 9, 11, 7, 3, 9]
    out = smp.apply_rep_penalty(row, hist, pen, 0, frac)
    fp, den = 1 << frac, (1 << frac) + pen
    for t in range(50):
        v = int(row[t])
        want = (v * fp // den if v >= 0 else v * den // fp) if t in set(hist) else v
        assert int(out[t]) == want
    # n = 3: prefix (7, 3) also occurs at i = 1 (7, 3 -> 9) and i = 5 (7, 3 -> end): 9 is banned
    ban = smp.apply_rep_penalty(row, hist + [7, 3], 0, 3, frac)
    assert int(ban[9]) == smp.NGRAM_BAN
    assert [t for t in range(50) if ban[t] != row[t]] == [9]
    assert np.array_equal(smp.apply_rep_penalty(row, [], pen, 3, frac), row)


def test_prng_word_sha256():
    assert hashlib.sha256(b"abc").hexdigest().startswith("ba7816bf8f01cfea")   # FIPS 180-2 B.1
    msg = smp.PRNG_TAG + (5).to_bytes(8, "big") + (9).to_bytes(8, "big") + (0).to_bytes(8, "big")
    assert len(msg) == 47
    assert smp.prng_word(5, 9, 0) == int(hashlib.sha256(msg).hexdigest()[:16], 16)
    assert smp.prng_word(-1, 0, 0) == smp.prng_word((1 << 64) - 1, 0, 0)          # low 64 bits of the seed


def test_lemire_closed_form():
    mask = (1 << 64) - 1
    for n in (2, 3, 7, 1000, 65537, (1 << 40) + 3, (1 << 63) + 5, (1 << 64) - 1):
        for seed, pos in ((0, 0), (1, 5), (99, 12345)):
            t = smp.draw_uniform_int(n, seed, pos)
            assert 0 <= t < n
            words = [smp.prng_word(seed, pos, j) for j in range(8)]
            thr = (1 << 64) % n
            j = next(j for j, w in enumerate(words) if ((w * n) & mask) >= thr)   # first word not rejected
            assert t == (words[j] * n) >> 64
    assert smp.draw_uniform_int(1, 3, 4) == 0 and smp.draw_uniform_int(0, 3, 4) == 0


def test_sample_token_modes():
    frac = 16
    row = (np.arange(40, dtype=np.int64) - 20) * 1500
    assert smp.sample_token(row, "greedy", frac) == 39
    tie = np.array([1, 5, 5, 2], dtype=np.int64)
    assert smp.sample_token(tie, "greedy", frac) == 1                              # numpy first-max
    # temperature identity: the probabilities are the plain softmax
    p = smp.probs(row, 1 << frac, frac)
    assert np.array_equal(p, softmax_rows(row[None, :], frac)[0])
    # seeded draws: reproducible, position- and seed-dependent on a flat row (test_bonsai_smoke.py:336-354)
    flat = np.zeros(200, dtype=np.int64)
    draw = lambda s: [smp.sample_token(flat, "top_p", frac, inv_temp=round(65536 / 0.6), top_k=20,
                                       top_p_fp=round(0.95 * 65536), seed=s, position=q) for q in range(16)]
    assert draw(0) == draw(0) and draw(999) != draw(0)
    assert all(t >= 180 for t in draw(0))                                          # top-20 keeps the high ids
    with pytest.raises(OverflowError):
        smp.sample_token(np.array([1 << 62, 0], dtype=np.int64), "temp", frac, inv_temp=4 << frac)
