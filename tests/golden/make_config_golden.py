#!/usr/bin/env python3
"""Write the oracle's digests of the five BASELINE configurations (tests/golden/configs.json).

Every input is regenerated from seeds by oracle/configs.py; every output is computed by the CPU oracle (the numpy
restatement with its pinned C twin, oracle/c). Nothing from the reference is imported or run.

  python tests/golden/make_config_golden.py            # C1-C4 (about a minute)
  python tests/golden/make_config_golden.py --c5       # also C5: 32 sequences x 64 greedy steps x 36 layers
                                                       # (about an hour on 8 cores; resumable, one sequence at a
                                                       # time, partial results in tests/golden/c5_partial.json)

C5 records every sequence's 64 greedy tokens and, per step, the SHA-256 of the batch's concatenated per-sequence
logits-row digests (oracle.configs.c5_step_digest).
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import configs as C  # noqa: E402

OUT = HERE / "configs.json"
PARTIAL = HERE / "c5_partial.json"


def c1_c4() -> dict:
    res = {}
    t = time.time()
    o = C.c1_oracle()
    res["c1"] = {"out_sha256": C.sha(o["out"]), "out_head": [int(v) for v in o["out"][0, :4]]}
    o = C.c2_oracle()
    res["c2"] = {"ctx": C.C2_CTX, "out_sha256": C.sha(o["out"]), "k_new_sha256": C.sha(o["k_new"]),
                 "v_new_sha256": C.sha(o["v_new"])}
    o = C.c3_oracle()
    res["c3"] = {"T": C.C3_T, "out_sha256": C.sha(o["out"]), "k_sha256": C.sha(o["k"]), "v_sha256": C.sha(o["v"])}
    o = C.c4_oracle()
    res["c4"] = {**C.C4, "out_sha256": C.sha(o["out"]), "sel_sha256": C.sha(o["sel"].astype("int64"))}
    print(f"C1-C4 in {time.time() - t:.1f} s", flush=True)
    return res


def c5() -> dict:
    part = json.loads(PARTIAL.read_text()) if PARTIAL.exists() else {}
    lens, first, _ = C.c5_spec()
    model = C.c5_model()
    bufs = C.c5_buffers()
    steps = C.C5["steps"]
    for b in range(C.C5["B"]):
        if str(b) in part:
            continue
        t = time.time()
        toks, digs = C.c5_sequence(model, b, steps, bufs)
        part[str(b)] = {"tokens": toks, "row_sha256": digs}
        PARTIAL.write_text(json.dumps(part))
        print(f"C5 sequence {b} (context {int(lens[b])}) in {time.time() - t:.1f} s", flush=True)
    B = C.C5["B"]
    return {**C.C5, "lens": [int(v) for v in lens], "first": [int(v) for v in first],
            "tokens": [part[str(b)]["tokens"] for b in range(B)],
            "step_sha256": [C.c5_step_digest([part[str(b)]["row_sha256"][s] for b in range(B)])
                            for s in range(steps)]}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--c5", action="store_true")
    a = ap.parse_args()
    res = json.loads(OUT.read_text()) if OUT.exists() else {}
    res.update(c1_c4())
    OUT.write_text(json.dumps(res, indent=1) + "\n")
    if a.c5:
        res["c5"] = c5()
        OUT.write_text(json.dumps(res, indent=1) + "\n")
        PARTIAL.unlink()


if __name__ == "__main__":
    main()
