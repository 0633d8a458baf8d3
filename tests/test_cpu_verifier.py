"""The host (CPU) receipt verifier (integer_inference_engine_amd/verify.py ``CpuVerifier``: imie_cpu_forward and
imie_cpu_sample_token) against the oracle, on CPU only: the verifier role of bonsai/src/trinote/infer_int/verify.py
:156-272 re-derived without the GPU. Its teacher-forced logits equal the oracle forward byte for byte, its sampler
equals the oracle sampler (pinned to the reference's truncation KATs in tests/test_oracle_sampler.py) over every
mode with penalties, honest turns verify under every strategy with the reference's digests, and forged tokens are
caught at their position."""
import hashlib
from types import SimpleNamespace

import numpy as np
import pytest

from oracle import bonsai_model as obm
from oracle import sampler as smp
from oracle.q1 import q1_rows

FRAC = 16


def _digest(row):
    return hashlib.sha256(np.ascontiguousarray(row, dtype="<i8").tobytes()).hexdigest()


def _cfg(mode, **kw):
    base = dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, seed=0, rep_penalty=0, no_repeat_ngram=0)
    base.update(kw)
    return SimpleNamespace(mode=mode, **base)


def _oracle_rows(model, ids):
    c = {"H": model["cfg"]["H"], "Hkv": model["cfg"]["Hkv"], "hd": model["cfg"]["hd"]}
    x = q1_rows(*model["embed"], ids)
    for layer in model["layers"]:
        x = obm.layer_forward(x, layer, c, model["cos"], model["sin"], FRAC, None, None, 0)[0]
    return obm.head_logits(model, x, FRAC)


def _pick(cfg):
    from integer_inference_engine_amd.sampler_gpu import config_c
    c = config_c(cfg, FRAC)

    def pick(row, position, hist):
        return smp.sample_token(row, cfg.mode, FRAC, inv_temp=c.inv_temp, top_k=c.top_k, top_p_fp=c.top_p,
                                min_p_fp=c.min_p, seed=cfg.seed, position=position, hist=hist,
                                rep_penalty=cfg.rep_penalty, no_repeat_ngram=cfg.no_repeat_ngram)
    return pick


def _produce(model, input_ids, n, cfg, eff):
    seq, rows = list(input_ids), []
    pick = _pick(cfg)
    for _ in range(n):
        row = _oracle_rows(model, seq[-eff:])[-1]
        rows.append(row)
        seq.append(pick(row, len(seq), list(seq)))
    return seq[len(input_ids):], rows


@pytest.fixture(scope="module")
def cpu_verifier(tmp_path_factory):
    from integer_inference_engine_amd import artifact as A
    from integer_inference_engine_amd.verify import CpuVerifier
    from tests.gguf_writer import artifact_model, bonsai_gguf
    p = tmp_path_factory.mktemp("cv") / "b.gguf"
    bonsai_gguf(p, seed=41, ctx=48)
    art = A.import_gguf(p)
    v = CpuVerifier(art, threads=4)
    yield v, artifact_model(art)
    v.close()


def test_host_forward_equals_oracle(cpu_verifier):
    v, model = cpu_verifier
    for ids in ([3], [9, 10, 11, 200, 3], list(range(40, 88))):
        got = v.logits_dev(ids)
        assert np.array_equal(got, _oracle_rows(model, ids)), len(ids)
        assert np.array_equal(v.logits_dev(ids, last_only=True)[0], got[-1])
    with pytest.raises(ValueError):
        v.logits_dev(list(range(49)))                              # beyond the 48-row RoPE window
    with pytest.raises(ValueError):
        v.logits_dev([0, 256])                                     # outside the vocabulary


@pytest.mark.parametrize("mode,kw", [("greedy", {}), ("greedy", dict(rep_penalty=13107, no_repeat_ngram=2)),
                                     ("temp", dict(temperature=0.7, seed=5)),
                                     ("top_k", dict(temperature=0.9, top_k=7, seed=11, rep_penalty=6553)),
                                     ("top_p", dict(temperature=0.6, top_k=20, top_p=0.95, seed=3)),
                                     ("top_p", dict(temperature=1.3, top_p=0.5, seed=9, no_repeat_ngram=3)),
                                     ("min_p", dict(temperature=0.8, min_p=0.15, seed=31))])
def test_host_sampler_equals_oracle(mode, kw):
    """Fuzzed rows with ties, negative and large logits, short and repetitive histories."""
    from integer_inference_engine_amd import _lib
    from integer_inference_engine_amd.sampler_gpu import config_c
    import ctypes
    so = _lib.lib()
    cfg = _cfg(mode, **kw)
    c = config_c(cfg, FRAC)
    pick = _pick(cfg)
    rng = np.random.default_rng(len(mode) * 7 + len(kw))
    for trial in range(40):
        V = int(rng.integers(2, 400))
        row = rng.integers(-(1 << 20), 1 << 20, size=V).astype(np.int64)
        if trial % 3 == 0:
            row[rng.integers(0, V, size=V // 3)] = row.max()              # ties at the top
        hist = [int(v) for v in rng.integers(0, V, size=int(rng.integers(0, 12)))]
        if trial % 4 == 0 and len(hist) > 3:
            hist = hist[:2] * 4                                            # repeated n-grams
        pos = int(rng.integers(0, 1 << 30))
        hh = np.ascontiguousarray(np.asarray(hist, dtype=np.int64))
        tok = ctypes.c_int64()
        rc = so.imie_cpu_sample_token(row.ctypes.data, V, ctypes.byref(c), hh.ctypes.data if hh.size else None,
                                      hh.size, pos, ctypes.byref(tok))
        assert rc == 0
        assert tok.value == pick(row, pos, hist), (trial, V)


def test_greedy_turn_verifies_and_forgery_is_caught(cpu_verifier):
    from integer_inference_engine_amd import verify as V
    v, model = cpu_verifier
    inp = [9, 10, 11, 200, 3]
    out, rows = _produce(model, inp, 7, _cfg("greedy"), v.eff)
    res = V.verify_greedy(v, inp, out)
    assert res["ok"] and res["strategy"] == "greedy-full" and res["checked"] == 7
    assert [p["logitsDigest"] for p in res["positions"]] == [_digest(r) for r in rows]
    bad = list(out)
    bad[3] = (bad[3] + 1) % 256
    res = V.verify_greedy(v, inp, bad)
    assert not res["ok"] and [p["match"] for p in res["positions"]].index(False) == 3
    ch = V.challenge_position(v, inp, out, 2)
    assert ch["match"] and ch["logitsDigest"] == _digest(rows[2])
    aud = V.verify_sampled(v, inp, out, k=3, seed=4)
    assert aud["ok"] and aud["checked"] == 3


def test_sliding_window_and_resample(cpu_verifier):
    from integer_inference_engine_amd import verify as V
    v, model = cpu_verifier
    inp = [int(t) for t in np.arange(44) % 256]
    out, rows = _produce(model, inp, 8, _cfg("greedy"), v.eff)        # 52 tokens > the 48-position window
    res = V.verify_greedy(v, inp, out)
    assert res["ok"] and res["strategy"] == "greedy-sliding"
    assert [p["logitsDigest"] for p in res["positions"]] == [_digest(r) for r in rows]
    cfg = _cfg("top_p", temperature=0.6, top_k=20, top_p=0.95, seed=3, rep_penalty=13107)
    inp2 = [4, 8, 15, 16]
    out2, _ = _produce(model, inp2, 6, cfg, v.eff)
    assert V.verify_resample(v, inp2, out2, sampler_cfg=cfg)["ok"]
    bad = list(out2)
    bad[4] = (bad[4] + 1) % 256
    assert [p["match"] for p in V.verify_resample(v, inp2, bad, sampler_cfg=cfg)["positions"]].index(False) == 4
    v.receipt_verify_strategy = "cached-replay"
    try:
        with pytest.raises(ValueError, match="no exact cached generator"):
            V.verify_greedy(v, inp2, out2)
    finally:
        v.receipt_verify_strategy = "auto"
