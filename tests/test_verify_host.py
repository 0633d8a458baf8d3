"""Host logic of the receipt verifier (integer_inference_engine_amd/verify.py) on CPU: strategy selection
(verify.py:60-103), replay bookkeeping (:106-117), the explicit cached-replay window refusal (:165-169) and the
empty-turn results, with stand-in models (no device work is reached)."""
from types import SimpleNamespace

import pytest

from integer_inference_engine_amd import verify as V


def _model(threshold=None, strategy="auto", replay=True, eff=16):
    m = SimpleNamespace(receipt_verify_cached_threshold=threshold, receipt_verify_strategy=strategy, eff=eff,
                        cfg={"frac": 16})
    if replay:
        m.replay = lambda *a, **k: None
    return m


def test_strategy_selection_follows_the_reference():
    assert V._strategy(_model(), 500) == "teacher-forced"                 # no threshold: never replays
    assert V._strategy(_model(threshold=64), 63) == "teacher-forced"
    assert V._strategy(_model(threshold=64), 64) == "cached-replay"
    assert V._strategy(_model(threshold=0), 1) == "cached-replay"         # clamped to >= 1
    assert V._strategy(_model(threshold=1, strategy="teacher-forced"), 99) == "teacher-forced"
    assert V._strategy(_model(strategy="cached-replay"), 1) == "cached-replay"
    with pytest.raises(ValueError, match="no exact cached generator"):
        V._strategy(_model(strategy="cached-replay", replay=False), 1)
    with pytest.raises(ValueError, match="unknown receipt verification strategy"):
        V._strategy(_model(strategy="fastest"), 1)
    assert V._strategy(_model(threshold=4, replay=False), 10) == "teacher-forced"   # no replay: never selected


def test_cached_window_rules():
    m = _model(strategy="cached-replay", eff=8)
    assert V._check_cached(m, list(range(8)), "cached-replay") is True
    with pytest.raises(ValueError, match="exceeds the exact context window"):
        V._check_cached(m, list(range(9)), "cached-replay")
    auto = _model(threshold=1, eff=8)
    assert V._check_cached(auto, list(range(9)), "cached-replay") is False      # auto falls back to teacher-forced
    assert V._check_cached(auto, list(range(4)), "teacher-forced") is False


def test_replay_positions_and_empty_turns():
    ok, pos = V._replay_positions([5, 6], [7, 8, 9], [7, 1, 9])
    assert not ok and [p["match"] for p in pos] == [True, False, True] and pos[0]["position"] == 2
    ok, pos = V._replay_positions([5], [7, 8], [7])                              # short replay fails closed
    assert not ok and pos[1]["predicted"] is None
    m = _model()
    assert V.verify_greedy(m, [1, 2], []) == {"ok": True, "checked": 0, "positions": [], "strategy": "greedy-full"}
    assert V.verify_resample(m, [1], [], sampler_cfg=None)["strategy"] == "resample-full"
    assert V.verify_sampled(m, [1], [], k=3) == {"ok": True, "checked": 0, "positions": [],
                                                 "strategy": "greedy-sampled"}
    with pytest.raises(IndexError):
        V.challenge_position(m, [1], [2], 1)


def test_host_logits_digest_is_sha256_of_le_int64():
    import hashlib
    import numpy as np
    row = np.array([1, -2, 1 << 62], dtype=np.int64)
    assert V.logits_digest(row) == hashlib.sha256(row.astype("<i8").tobytes()).hexdigest()
