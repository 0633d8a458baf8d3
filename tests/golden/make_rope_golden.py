"""Write tests/golden/rope_yarn_8b.json: the sha256 (little-endian int64 cos then sin) of the Bonsai-8B YaRN
table for 4160 and 32832 positions, from the oracle restatement, plus a few rows in clear.

The fixture freezes the table bytes the device path reads; the oracle builder itself is pinned by the
reference's KAT rows (bonsai/tests/test_bonsai_smoke.py:91-107). Run: python tests/golden/make_rope_golden.py
"""
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle.rope import bonsai8b_tables, table_hash  # noqa: E402

out = {}
for n in (4160, 32832):
    cos, sin = bonsai8b_tables(n)
    out[str(n)] = {"sha256": table_hash(cos, sin),
                   "rows": {str(p): {"cos": cos[p].tolist(), "sin": sin[p].tolist()} for p in (1, 777, n - 1)}}
(Path(__file__).parent / "rope_yarn_8b.json").write_text(json.dumps(out, indent=1) + "\n")
