"""Receipt re-execution on the device (integer_inference_engine_amd/verify.py) against turns produced by the oracle.

Gates after bonsai/src/trinote/infer_int/verify.py:156-272 and bonsai/tests/test_bonsai_smoke.py:202-285: an
honest greedy / penalized / seeded-sampler turn verifies under every strategy (teacher-forced full, sliding
window, sampled audit, challenge, cached replay), every position's logitsDigest equals SHA-256 of the oracle's
row, and a forged token is caught at its position."""
import hashlib
from types import SimpleNamespace

import numpy as np
import pytest

from oracle import bonsai_model as obm
from oracle import sampler as smp
from oracle.q1 import q1_rows

pytestmark = pytest.mark.gpu
FRAC = 16


def _digest(row):
    return hashlib.sha256(np.ascontiguousarray(row, dtype="<i8").tobytes()).hexdigest()


@pytest.mark.parametrize("rows,vocab,ld", [(1, 151936, 151936), (70, 151936, 151936), (5, 7, 7), (9, 15, 17),
                                           (66, 8, 8), (3, 1, 1), (2, 4099, 4100)])
def test_logits_digest_dev_matches_sha256(gpu, rows, vocab, ld):
    import torch
    from integer_inference_engine_amd.verify import logits_digest_dev
    rng = np.random.default_rng(rows * 1000 + vocab)
    full = rng.integers(-(1 << 62), 1 << 62, size=(rows, ld), dtype=np.int64)
    dev = torch.from_numpy(full).cuda()[:, :vocab]
    assert logits_digest_dev(dev) == [_digest(full[r, :vocab]) for r in range(rows)]


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
    """The oracle producer: each token from the last row of the clamped window, history = the whole sequence."""
    seq, rows = list(input_ids), []
    pick = _pick(cfg)
    for _ in range(n):
        row = _oracle_rows(model, seq[-eff:])[-1]
        rows.append(row)
        seq.append(pick(row, len(seq), list(seq)))
    return seq[len(input_ids):], rows


@pytest.fixture(scope="module")
def verifier(tmp_path_factory):
    from integer_inference_engine_amd import artifact as A
    from integer_inference_engine_amd.verify import DeviceVerifier
    from tests.gguf_writer import artifact_model, bonsai_gguf
    p = tmp_path_factory.mktemp("v") / "b.gguf"
    bonsai_gguf(p, seed=41, ctx=48)
    art = A.import_gguf(p)
    v = DeviceVerifier(art)
    yield v, artifact_model(art)
    v.close()


def test_greedy_turn_verifies_and_forgery_is_caught(verifier):
    from integer_inference_engine_amd import verify as V
    v, model = verifier
    inp = [9, 10, 11, 200, 3]
    out, rows = _produce(model, inp, 7, _cfg("greedy"), v.eff)
    res = V.verify_greedy(v, inp, out)
    assert res["ok"] and res["strategy"] == "greedy-full" and res["checked"] == 7
    assert [p["logitsDigest"] for p in res["positions"]] == [_digest(r) for r in rows]
    assert [p["position"] for p in res["positions"]] == list(range(5, 12))
    bad = list(out)
    bad[3] = (bad[3] + 1) % 256
    res = V.verify_greedy(v, inp, bad)
    assert not res["ok"] and [p["match"] for p in res["positions"]].index(False) == 3
    for i in range(len(out)):
        ch = V.challenge_position(v, inp, out, i)
        assert ch["match"] and ch["predicted"] == out[i] and ch["logitsDigest"] == _digest(rows[i])
    assert V.verify_greedy(v, inp, []) == {"ok": True, "checked": 0, "positions": [], "strategy": "greedy-full"}
    with pytest.raises(ValueError, match="non-empty prompt"):
        V.verify_greedy(v, [], out)
    with pytest.raises(IndexError):
        V.challenge_position(v, inp, out, len(out))


def test_sampled_audit_uses_the_reference_selection(verifier):
    from integer_inference_engine_amd import verify as V
    v, model = verifier
    inp = [1, 2, 3]
    out, rows = _produce(model, inp, 9, _cfg("greedy"), v.eff)
    res = V.verify_sampled(v, inp, out, k=4, seed=7)
    chosen = sorted(int(j) for j in np.random.Generator(np.random.Philox(key=7)).choice(9, size=4, replace=False))
    assert res["ok"] and res["checked"] == 4 and res["of"] == 9 and res["strategy"] == "greedy-sampled"
    assert [p["position"] - 3 for p in res["positions"]] == chosen
    assert [p["logitsDigest"] for p in res["positions"]] == [_digest(rows[i]) for i in chosen]
    v.DIGEST_DEVICE_MIN_ROWS = 1                                 # the device digest path on the same rows
    try:
        again = V.verify_sampled(v, inp, out, k=4, seed=7)
    finally:
        v.DIGEST_DEVICE_MIN_ROWS = 64
    assert again == res


def test_penalized_greedy_and_sliding_window(verifier):
    from integer_inference_engine_amd import verify as V
    v, model = verifier
    cfg = _cfg("greedy", rep_penalty=13107, no_repeat_ngram=2)
    inp = [5, 6, 7, 5, 6]
    out, _ = _produce(model, inp, 8, cfg, v.eff)
    res = V.verify_greedy(v, inp, out, rep_penalty_fp=13107, no_repeat_ngram=2)
    assert res["ok"] and res["strategy"] == "greedy-full"
    long_inp = [int(t) for t in np.random.default_rng(3).integers(0, 256, size=v.eff - 3)]
    out, rows = _produce(model, long_inp, 6, cfg, v.eff)         # crosses the window: sliding
    res = V.verify_greedy(v, long_inp, out, rep_penalty_fp=13107, no_repeat_ngram=2)
    assert res["ok"] and res["strategy"] == "greedy-sliding"
    assert [p["logitsDigest"] for p in res["positions"]] == [_digest(r) for r in rows]


@pytest.mark.parametrize("cfg", [_cfg("top_k", temperature=0.7, top_k=7, seed=23),
                                 _cfg("top_p", temperature=0.6, top_k=20, top_p=0.95, seed=3, rep_penalty=13107),
                                 _cfg("min_p", temperature=0.9, min_p=0.15, seed=31, no_repeat_ngram=2)])
def test_resample_verifies_seeded_turns(verifier, cfg):
    from integer_inference_engine_amd import verify as V
    v, model = verifier
    inp = [40, 41, 42, 43]
    out, _ = _produce(model, inp, 8, cfg, v.eff)
    res = V.verify_resample(v, inp, out, sampler_cfg=cfg)
    assert res["ok"] and res["strategy"] == "resample-full", res
    bad = list(out)
    bad[2] = (bad[2] + 1) % 256
    forged = V.verify_resample(v, inp, bad, sampler_cfg=cfg)
    assert not forged["ok"] and [p["match"] for p in forged["positions"]].index(False) == 2


def test_cached_replay_strategies(verifier):
    from integer_inference_engine_amd import verify as V
    v, model = verifier
    inp = [12, 13, 14]
    greedy_out, _ = _produce(model, inp, 6, _cfg("greedy"), v.eff)
    pen = _cfg("greedy", rep_penalty=13107, no_repeat_ngram=2)
    pen_out, _ = _produce(model, inp, 6, pen, v.eff)
    samp = _cfg("top_k", temperature=0.8, top_k=9, seed=5)
    samp_out, _ = _produce(model, inp, 6, samp, v.eff)
    assert v.receipt_verify_cached_threshold is None                     # "auto" never replays on the device
    assert V.verify_greedy(v, inp, greedy_out * 6)["strategy"] == "greedy-full"
    v.receipt_verify_strategy = "cached-replay"                            # explicit replay, no threshold
    assert V.verify_greedy(v, inp, greedy_out)["strategy"] == "greedy-cached-replay"
    v.receipt_verify_strategy = "auto"
    v.receipt_verify_cached_threshold = 1
    try:
        res = V.verify_greedy(v, inp, greedy_out)
        assert res["ok"] and res["strategy"] == "greedy-cached-replay" and res["logitsDigest"] is None
        assert V.verify_greedy(v, inp, pen_out, rep_penalty_fp=13107, no_repeat_ngram=2)["ok"]
        res = V.verify_resample(v, inp, samp_out, sampler_cfg=samp)
        assert res["ok"] and res["strategy"] == "resample-cached-replay"
        bad = list(greedy_out)
        bad[-1] = (bad[-1] + 1) % 256
        assert not V.verify_greedy(v, inp, bad)["ok"]
        v.receipt_verify_strategy = "teacher-forced"
        assert V.verify_greedy(v, inp, greedy_out)["strategy"] == "greedy-full"
        v.receipt_verify_strategy = "cached-replay"
        with pytest.raises(ValueError, match="exceeds the exact context window"):
            V.verify_greedy(v, list(range(v.eff)), greedy_out)
    finally:
        v.receipt_verify_cached_threshold = None
        v.receipt_verify_strategy = "auto"


def test_device_turn_verifies_on_the_host_verifier(verifier):
    """A greedy turn generated by the device decode loop, re-derived by the independent host verifier
    (CpuVerifier): the receipt check needs no trust in the GPU."""
    from integer_inference_engine_amd import verify as V
    from integer_inference_engine_amd.verify import CpuVerifier
    v, model = verifier
    inp = [7, 77, 177]
    out = v.replay(inp, 9)
    host = CpuVerifier(v.artifact, threads=8)
    try:
        res = V.verify_greedy(host, inp, out)
        assert res["ok"] and res["checked"] == 9
        dev = V.verify_greedy(v, inp, out)
        assert [p["logitsDigest"] for p in res["positions"]] == [p["logitsDigest"] for p in dev["positions"]]
    finally:
        host.close()
