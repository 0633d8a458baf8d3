"""Host-side sampler config rules (integer_inference_engine_amd/sampler_gpu.py) on CPU, against
validate_sampler_config (bonsai/src/trinote/infer_int/sampler.py:71-91) and the modes that read the nucleus
threshold (sampler.py:403-437: only top_k / top_p pass it to _truncate)."""
from types import SimpleNamespace

import pytest

from integer_inference_engine_amd import sampler_gpu as S


def _cfg(mode, **kw):
    base = dict(mode=mode, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, seed=0, rep_penalty=0,
                no_repeat_ngram=0)
    base.update(kw)
    return SimpleNamespace(**base)


def test_unused_top_p_is_ignored_outside_nucleus_modes():
    for mode in ("temp", "min_p"):
        for tp in (0.0, -1.0, 1.5, 7.0):
            c = S.config_c(_cfg(mode, top_p=tp, min_p=0.1), 16)
            assert c.top_p == 1 << 16                       # no truncation whatever the field held
    assert S.config_c(_cfg("greedy", top_p=3.0), 16).top_p == 1 << 16


def test_top_p_is_validated_and_passed_in_nucleus_modes():
    with pytest.raises(ValueError, match="top_p must be in"):
        S.config_c(_cfg("top_p", top_p=1.5), 16)
    with pytest.raises(ValueError, match="top_p must be in"):
        S.config_c(_cfg("top_p", top_p=0.0), 16)
    assert S.config_c(_cfg("top_p", top_p=0.5), 16).top_p == 1 << 15
    assert S.config_c(_cfg("top_k", top_k=20, top_p=0.95), 16).top_p == round(0.95 * 65536)


def test_temperature_is_checked_even_with_committed_integers():
    cfg = _cfg("temp", temperature=0.0)
    cfg.inv_temp_fp_committed = 65536
    with pytest.raises(ValueError, match="temperature must be > 0"):
        S.config_c(cfg, 16)
    cfg.temperature = 0.7                                      # committed int wins over the float when valid
    assert S.config_c(cfg, 16).inv_temp == 65536
