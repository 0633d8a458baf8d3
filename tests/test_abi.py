"""The C-ABI library loads, exports every declared symbol, and its host-side repack is correct (CPU only)."""
import ctypes
import re
from pathlib import Path

import numpy as np

from integer_inference_engine_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        for m in re.finditer(r"^\s*(?:[A-Za-z_][\w\s\*]*?)\b((?:bonsai|qk|imie)_\w+)\s*\(", h.read_text(), re.M):
            names.add(m.group(1))
    return names


def test_library_loads_and_exports_declared_symbols():
    so = _lib.lib()
    declared = _declared_symbols()
    assert declared, "no declarations found in include/*.h"
    missing = [n for n in sorted(declared) if not hasattr(so, n)]
    assert not missing, f"symbols declared in include/*.h but not exported: {missing}"
    assert set(_lib.SIGNATURES) <= declared, sorted(set(_lib.SIGNATURES) - declared)


def test_q1_repack_host_layout():
    so = _lib.lib()
    rng = np.random.default_rng(0)
    N, nb = 37, 6                      # ragged: pads rows to 48 and blocks to 8
    bits = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    scale = rng.integers(-(1 << 30), 1 << 30, size=(N, nb), dtype=np.int64)
    ntiles, nslabs = 3, 2
    bt = np.zeros((ntiles, nslabs, 64, 16), dtype=np.uint8)
    st = np.zeros((ntiles, nslabs, 64), dtype=np.int32)
    rc = so.imie_q1_repack_host(bits.ctypes.data, scale.ctypes.data, N, nb, 0, bt.ctypes.data, st.ctypes.data)
    assert rc == 0
    for tile in range(ntiles):
        for sl in range(nslabs):
            for lane in range(64):
                row, blk = tile * 16 + (lane & 15), sl * 4 + (lane >> 4)
                if row < N and blk < nb:
                    assert np.array_equal(bt[tile, sl, lane], bits[row, blk])
                    assert st[tile, sl, lane] == scale[row, blk]
                else:
                    assert not bt[tile, sl, lane].any() and st[tile, sl, lane] == 0
