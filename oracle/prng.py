"""Counter-based SplitMix64 streams for seeded synthetic inputs (test infrastructure).

Every element of every synthetic tensor is a pure function of ``(seed, tensor_id, index)``, so a test on the
GPU box can regenerate exactly the inputs a golden digest was computed from, at any size, without storing them.
This is our own generator (the reference draws with numpy ``default_rng``); pinned by the published SplitMix64
test vector in ``tests/test_oracle_core.py``.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def splitmix64(state: int, n: int) -> np.ndarray:
    """The first ``n`` outputs of SplitMix64 started at ``state`` (uint64)."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(state & 0xFFFFFFFFFFFFFFFF) + idx * _GAMMA
        return _mix(z)


def stream(seed: int, tensor_id: int, n: int) -> np.ndarray:
    """``n`` uint64 draws keyed by (seed, tensor_id)."""
    with np.errstate(over="ignore"):
        key = _mix(np.array([(seed * 0x100000001B3 + tensor_id * 0x9E3779B1 + 0x632BE59BD9B4E019)
                             & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64))[0]
    return splitmix64(int(key), n)


def uniform_int(seed: int, tensor_id: int, shape, lo: int, hi: int) -> np.ndarray:
    """int64 values in ``[lo, hi)`` (modulo-reduced; bias irrelevant for parity tests)."""
    shape = tuple(int(s) for s in np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
    n = int(np.prod(shape, dtype=np.int64)) if shape else 1
    span = hi - lo
    assert 0 < span <= (1 << 63)
    u = stream(seed, tensor_id, n)
    v = (u % np.uint64(span)).astype(np.int64) + np.int64(lo) if span < (1 << 63) else u.view(np.int64)
    return v.reshape(shape)


def uniform_bytes(seed: int, tensor_id: int, shape) -> np.ndarray:
    """uint8 values uniform in [0, 256)."""
    n = int(np.prod(shape, dtype=np.int64))
    words = stream(seed, tensor_id, (n + 7) // 8)
    return words.view(np.uint8)[:n].reshape(shape).copy()
