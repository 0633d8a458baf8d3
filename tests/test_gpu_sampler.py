"""Device integer samplers vs the oracle, token for token (the reference's sampler parity rung,
bonsai/tests/test_bonsai35_gpu.py:262-276: greedy with penalty + n-gram, temp, top_k, top_p, min_p)."""
import ctypes
from types import SimpleNamespace

import numpy as np
import pytest

from oracle import sampler as smp

pytestmark = pytest.mark.gpu
FRAC = 16


def _cfg(mode, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, seed=0, rep_penalty=0, no_repeat_ngram=0):
    return SimpleNamespace(mode=mode, temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p, seed=seed,
                           rep_penalty=rep_penalty, no_repeat_ngram=no_repeat_ngram)


def _oracle(row, cfg, position, hist):
    from integer_inference_engine_amd.sampler_gpu import config_c
    c = config_c(cfg, FRAC)
    return smp.sample_token(row, cfg.mode, FRAC, inv_temp=c.inv_temp, top_k=c.top_k, top_p_fp=c.top_p,
                            min_p_fp=c.min_p, seed=cfg.seed, position=position, hist=hist,
                            rep_penalty=cfg.rep_penalty, no_repeat_ngram=cfg.no_repeat_ngram)


CONFIGS = [
    _cfg("greedy", rep_penalty=13107, no_repeat_ngram=2),
    _cfg("temp", temperature=0.8, seed=19, rep_penalty=13107),
    _cfg("top_k", temperature=0.7, top_k=7, seed=23),
    _cfg("top_p", temperature=0.7, top_k=9, top_p=0.8, seed=29),
    _cfg("min_p", temperature=0.9, min_p=0.15, seed=31),
    _cfg("top_p", temperature=0.6, top_k=20, top_p=0.95, seed=0),          # qwen3-rec
    _cfg("top_p", temperature=1.3, top_k=0, top_p=0.5, seed=5),            # nucleus over the whole vocabulary
    _cfg("temp", temperature=1.0, seed=77),                                # identity temperature
]


@pytest.mark.parametrize("vocab", [7, 200, 4099, 151936])
@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_sample_token_matches_oracle(gpu, vocab, ci):
    from integer_inference_engine_amd.sampler_gpu import sample_token
    cfg = CONFIGS[ci]
    rng = np.random.default_rng(1000 * ci + vocab)
    hist = [int(t) for t in rng.integers(0, vocab, size=12)]
    hist += hist[-2:-1]                                                     # a repeated bigram prefix
    rows = [rng.integers(-(1 << 19), 1 << 19, size=vocab, dtype=np.int64),
            rng.integers(-4, 4, size=vocab, dtype=np.int64) * (1 << 14),     # heavy ties
            np.zeros(vocab, dtype=np.int64)]
    for ri, row in enumerate(rows):
        for pos in (0, 17, 4096):
            want = _oracle(row, cfg, pos, hist)
            got = sample_token(row, cfg, pos, FRAC, history_ids=hist)
            assert got == want, (ci, vocab, ri, pos)


def test_sample_token_guard_and_errors(gpu):
    from integer_inference_engine_amd.sampler_gpu import sample_token
    row = np.array([1 << 62, 0, 5], dtype=np.int64)
    with pytest.raises(OverflowError):
        sample_token(row, _cfg("temp", temperature=0.25), 0, FRAC)
    assert sample_token(row, _cfg("greedy"), 0, FRAC) == 0                 # greedy never scales
    with pytest.raises(ValueError):
        sample_token(row, _cfg("greedy", rep_penalty=5), 0, FRAC, history_ids=[9])   # token outside the vocab
    with pytest.raises(ValueError):
        sample_token(row, _cfg("top_k", top_k=0), 0, FRAC)


def test_draw_probe_matches_sha256_lemire(gpu):
    from integer_inference_engine_amd import _lib
    so = _lib.lib()
    rng = np.random.default_rng(5)
    totals = [0, 1, 2, 3, 65536, (1 << 47) + 11, (1 << 62) + 1, (1 << 63) - 1]
    totals += [int(t) for t in rng.integers(2, 1 << 40, size=20)]
    for total in totals:
        for seed, pos in ((0, 0), (7, 123), (-1, 5), (1 << 40, (1 << 33) + 7)):
            w, t = ctypes.c_uint64(), ctypes.c_int64()
            assert so.imie_sample_draw_probe(total, seed, pos, ctypes.byref(w), ctypes.byref(t)) == 0
            assert w.value == smp.prng_word(seed, pos, 0)
            assert t.value == smp.draw_uniform_int(total, seed, pos), (total, seed, pos)


def test_sample_rows_dev_matches_oracle(gpu):
    """Device rows with per-row positions and histories (the batched decode shape), twice in a row."""
    import torch
    from integer_inference_engine_amd.sampler_gpu import sample_rows_dev
    rng = np.random.default_rng(9)
    B, V, H = 5, 3001, 16
    cfg = _cfg("top_p", temperature=0.7, top_k=40, top_p=0.9, seed=3, rep_penalty=13107, no_repeat_ngram=3)
    for rep in range(2):
        logits = rng.integers(-(1 << 18), 1 << 18, size=(B, V), dtype=np.int64)
        pos = rng.integers(0, 10000, size=B, dtype=np.int64)
        hist = rng.integers(0, V, size=(B, H), dtype=np.int64)
        hlen = np.array([0, 3, H, 7, 1], dtype=np.int64)
        tok, status = sample_rows_dev(torch.from_numpy(logits).cuda(), cfg, FRAC, torch.from_numpy(pos).cuda(),
                                      torch.from_numpy(hist).cuda(), torch.from_numpy(hlen).cuda())
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        got = tok.cpu().numpy()
        for b in range(B):
            want = _oracle(logits[b], cfg, int(pos[b]), [int(t) for t in hist[b, :hlen[b]]])
            assert got[b] == want, (rep, b)
