"""The committed oracle digests of the BASELINE configurations (tests/golden/configs.json) are what the CPU oracle
computes today from the seeded inputs (CPU only; C5's 36-layer golden is too long to recompute here: its first
two steps of one sequence are, on four layers' worth of structure checked in tests/test_oracle_model.py)."""
import json
from pathlib import Path

import pytest

from oracle import configs as C

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "configs.json").read_text())


def test_c1_golden():
    assert C.sha(C.c1_oracle()["out"]) == GOLDEN["c1"]["out_sha256"]


def test_c2_golden():
    o = C.c2_oracle()
    g = GOLDEN["c2"]
    assert (C.sha(o["out"]), C.sha(o["k_new"]), C.sha(o["v_new"])) == (g["out_sha256"], g["k_new_sha256"],
                                                                         g["v_new_sha256"])


def test_c3_golden():
    o = C.c3_oracle()
    g = GOLDEN["c3"]
    assert (C.sha(o["out"]), C.sha(o["k"]), C.sha(o["v"])) == (g["out_sha256"], g["k_sha256"], g["v_sha256"])


def test_c4_golden():
    o = C.c4_oracle()
    assert C.sha(o["out"]) == GOLDEN["c4"]["out_sha256"]
    assert C.sha(o["sel"].astype("int64")) == GOLDEN["c4"]["sel_sha256"]


def test_c5_golden_shape():
    g = GOLDEN.get("c5")
    if g is None:
        pytest.skip("C5 golden not generated yet (tests/golden/make_config_golden.py --c5)")
    lens, first, _ = C.c5_spec()
    assert g["lens"] == [int(v) for v in lens] and g["first"] == [int(v) for v in first]
    assert len(g["tokens"]) == C.C5["B"] and all(len(t) == C.C5["steps"] for t in g["tokens"])
    assert len(g["step_sha256"]) == C.C5["steps"]
