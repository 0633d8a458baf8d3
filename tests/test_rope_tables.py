"""The product's host-side RoPE table builder (CPU only): reference KAT rows, equality with the oracle
restatement, and the committed table digest of the 8B shape."""
import json
from pathlib import Path

import numpy as np
import pytest

from integer_inference_engine_amd import rope_tables as rt
from oracle import rope as orope

GOLDEN = json.loads((Path(__file__).parent / "golden" / "rope_yarn_8b.json").read_text())


def test_product_yarn_kat_rows():
    # bonsai/tests/test_bonsai_smoke.py:91-107
    cos, sin = rt.bonsai8b_tables(2)
    assert (int(cos[0, 0]), int(sin[0, 0])) == (74_621, 0)
    assert (int(cos[1, 0]), int(sin[1, 0])) == (40_318, 62_792)
    assert (int(cos[1, 10]), int(sin[1, 10])) == (74_124, 8_598)
    assert (int(cos[1, 19]), int(sin[1, 19])) == (74_611, 1_235)


@pytest.mark.parametrize("n,hd,base", [(300, 64, 10000), (97, 128, 1_000_000), (1, 2, 10000)])
def test_product_plain_equals_oracle(n, hd, base):
    a = rt.plain_tables(n, hd, base)
    b = orope.build_rope_tables(n, hd, base)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


@pytest.mark.parametrize("ext", [1.0, 0.0, 0.5])
def test_product_yarn_equals_oracle(ext):
    kw = dict(base=500_000, freq_scale=0.125, n_ctx_orig=8192, ext_factor=ext, attn_factor=0.9)
    a = rt.yarn_tables(513, 64, **kw)
    b = orope.build_yarn_rope_tables(513, 64, **kw)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


@pytest.mark.parametrize("n", ["4160", "32832"])
def test_product_8b_table_matches_committed_digest(n):
    cos, sin = rt.bonsai8b_tables(int(n))
    assert orope.table_hash(cos, sin) == GOLDEN[n]["sha256"]
    for p, row in GOLDEN[n]["rows"].items():
        assert cos[int(p)].tolist() == row["cos"] and sin[int(p)].tolist() == row["sin"]
