"""gfx950 producer boundary for the Bonsai (Qwen3-dense, packed Q1_0) hot path.

Drop-in for ``bonsai/src/trinote/infer_int/gpu_native.py`` (reference interface, ``gpu_native.py:188-595``):
same function names, arguments and return conventions. Every result is byte-identical to the CPU integer
oracle; a nonzero library rc (envelope overflow, bad arguments) returns ``None`` exactly as the reference
wrapper does (``gpu_native.py:218-220``), so the reference model code keeps its own fallback policy.

Unlike the reference loader, a MISSING library is an error (``ImportError`` from ``_lib.lib()``): the hot path
never degrades silently to a CPU path inside this package. ``gpu_available()`` answers only whether a gfx950
device is usable.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

GROUP = 128
_L4_LO, _L4_HI = -2155905152, 2139062143   # balanced base-256 L=4 envelope (gpu_native.py:223)


def gpu_available() -> bool:
    """True iff the library loaded and a usable gfx950 GPU is present (gpu_native.py:188-190)."""
    return _lib.device_available()


def _dev() -> ctypes.CDLL | None:
    return _lib.lib() if _lib.device_available() else None


def _as_i64_2d(x) -> np.ndarray:
    return np.ascontiguousarray(np.atleast_2d(np.asarray(x, dtype=np.int64)))


def _scale_i64(scale_fp) -> np.ndarray:
    src = np.asarray(scale_fp)
    if not np.issubdtype(src.dtype, np.integer):
        raise TypeError(f"Q1_0 scale must be an integer dtype, got {src.dtype}")
    return np.ascontiguousarray(src, dtype=np.int64)


def q1_apply_gpu(x_fp: np.ndarray, bits: np.ndarray, scale_fp: np.ndarray, frac: int) -> "np.ndarray | None":
    """Packed-Q1_0 ``x @ W.T`` with a per-call weight upload (gpu_native.py:193-220)."""
    lib = _dev()
    if lib is None:
        return None
    x = _as_i64_2d(x_fp)
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint8))
    s = _scale_i64(scale_fp)
    out_f, n_blocks = s.shape
    if x.shape[1] != n_blocks * GROUP:
        raise ValueError(f"Q1_0 contraction mismatch: x has {x.shape[1]}, weight expects {n_blocks * GROUP}")
    out = np.empty((x.shape[0], out_f), dtype=np.int64)
    rc = lib.bonsai_q1_linear_gpu(x.ctypes.data, b.ctypes.data, s.ctypes.data, x.shape[0], int(out_f),
                                  int(n_blocks), int(frac), out.ctypes.data)
    return None if rc != 0 else out


def q1_apply_dp4a_gpu(x_fp, bits, scale_fp, frac: int, L: "int | None" = None) -> "np.ndarray | None":
    """Limb-decomposed Q1 apply (gpu_native.py:226-261). On gfx950 every Q1 apply already runs over balanced
    base-256 limbs on int8 MFMA, so this is the same kernel; an explicit L=4 outside the L=4 envelope raises
    as in the reference."""
    x = _as_i64_2d(x_fp)
    if L is not None and int(L) == 4 and x.size:
        mn, mx = int(x.min()), int(x.max())
        if not (_L4_LO <= mn and mx <= _L4_HI):
            raise ValueError(f"q1_apply_dp4a_gpu: explicit L=4 requires activations in [{_L4_LO}, {_L4_HI}], "
                             f"got [{mn}, {mx}]")
    return q1_apply_gpu(x, bits, scale_fp, frac)


def residency_available() -> bool:
    return _dev() is not None


def q1_register_weight(bits: np.ndarray, scale_fp: np.ndarray, *, gpu_coalesced: bool = False,
                       gpu_bmma: bool = False) -> "int | None":
    """Upload bits + scale once; return a handle >= 0 or None (gpu_native.py:270-306). The weight is stored in
    the gfx950 tile layout; scales are narrowed to int32 on device when lossless. ``gpu_coalesced`` /
    ``gpu_bmma`` select CUDA-specific layouts in the reference and are accepted for interface parity."""
    lib = _dev()
    if lib is None:
        return None
    if gpu_coalesced and gpu_bmma:
        raise ValueError("choose one GPU Q1 runtime layout")
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint8))
    src = np.asarray(scale_fp)
    if not np.issubdtype(src.dtype, np.integer):
        raise TypeError(f"Q1_0 scale must be an integer dtype, got {src.dtype}")
    if src.dtype.itemsize <= 4:
        s = np.ascontiguousarray(src, dtype=np.int32)
        h = lib.bonsai_q1_register_weight_i32(b.ctypes.data, s.ctypes.data, int(s.shape[0]), int(s.shape[1]))
    else:
        s = np.ascontiguousarray(src, dtype=np.int64)
        h = lib.bonsai_q1_register_weight(b.ctypes.data, s.ctypes.data, int(s.shape[0]), int(s.shape[1]))
    return None if int(h) < 0 else int(h)


def q1_apply_resident(handle: int, x_fp: np.ndarray, out_features: int, n_blocks: int,
                      frac: int) -> "np.ndarray | None":
    """Apply a registered weight to host activations (gpu_native.py:364-380)."""
    lib = _dev()
    if lib is None:
        return None
    x = _as_i64_2d(x_fp)
    if x.shape[1] != int(n_blocks) * GROUP:
        raise ValueError(f"Q1_0 contraction mismatch: x has {x.shape[1]}, weight expects {int(n_blocks) * GROUP}")
    out = np.empty((x.shape[0], int(out_features)), dtype=np.int64)
    rc = lib.bonsai_q1_apply_resident(int(handle), x.ctypes.data, x.shape[0], int(frac), out.ctypes.data)
    return None if rc != 0 else out


def q1_free_weights() -> None:
    lib = _dev()
    if lib is not None:
        lib.bonsai_q1_free_weights()


def gpu_memory_info() -> "dict[str, int] | None":
    """Allocator-visible device memory and the resident Q1 weight bytes (gpu_native.py:309-331)."""
    lib = _dev()
    if lib is None:
        return None
    free = ctypes.c_uint64()
    total = ctypes.c_uint64()
    if lib.bonsai_gpu_mem_info(ctypes.byref(free), ctypes.byref(total)) != 0:
        return None
    return {
        "free_bytes": int(free.value),
        "total_bytes": int(total.value),
        "used_bytes": int(total.value - free.value),
        "resident_weight_bytes": int(lib.bonsai_q1_resident_weight_bytes()),
    }
