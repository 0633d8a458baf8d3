"""gfx950 producer boundary for the north-mini-code Q4_K / Q6_K hot path.

Mirrors ``north-mini-code/src/nmc/qk_cuda.py`` (functions ``available``, ``qk_linear``, ``register_weight``,
``apply_resident``, ``apply_resident_grouped``, ``apply_resident_dp4a``, ``moe_ffn``, ``moe_ffn_batched``,
``free_all``, ``resident_count``, ``limbs_needed`` ...; qk_cuda.py:226-1124) with the same arguments and return
conventions: ``None`` on a library rc != 0, ``CudaRegistrationError`` when a registration fails. Calls are
serialized by a process lock as in the reference (qk_cuda.py:35-38).
"""
from __future__ import annotations

import ctypes
import threading

import numpy as np

from . import _lib

Q4_K, Q6_K = 0, 1
_LOCK = threading.RLock()
_BS = {Q4_K: 144, Q6_K: 210}


class CudaRegistrationError(RuntimeError):
    """A resident weight could not be committed to the device registry (qk_cuda.py:75-76)."""


def _dev():
    return _lib.lib() if _lib.device_available() else None


def available() -> bool:
    return _dev() is not None


def _require_weight_bytes(weight_raw, out_f: int, n_blocks: int, qtype: int) -> None:
    if qtype not in _BS:
        raise ValueError(f"unknown qtype {qtype}")
    need = int(out_f) * int(n_blocks) * _BS[qtype]
    if len(weight_raw) < need:
        raise ValueError(f"weight buffer has {len(weight_raw)} bytes, need {need}")


def _raw(weight_raw) -> np.ndarray:
    if isinstance(weight_raw, np.ndarray):
        return np.ascontiguousarray(weight_raw.reshape(-1).view(np.uint8))
    return np.frombuffer(bytes(weight_raw), dtype=np.uint8)


def qk_linear(weight_raw, x_int: np.ndarray, out_f: int, n_blocks: int, fw: int, qtype: int):
    """y[t, o] = (sum_i W[o, i] x[t, i]) >> fw from raw blocks (qk_cuda.py:230-244)."""
    lib = _dev()
    if lib is None:
        return None
    x = np.ascontiguousarray(np.atleast_2d(np.asarray(x_int, dtype=np.int64)))
    T, in_f = x.shape
    assert in_f == n_blocks * 256, (in_f, n_blocks)
    _require_weight_bytes(weight_raw, out_f, n_blocks, qtype)
    w = _raw(weight_raw)
    out = np.empty((T, out_f), dtype=np.int64)
    with _LOCK:
        rc = lib.qk_linear_cuda(w.ctypes.data, x.ctypes.data, T, out_f, n_blocks, int(fw), int(qtype), out.ctypes.data)
    return None if rc != 0 else out


def resident_available() -> bool:
    return available()


def register_weight(weight_raw, out_f: int, n_blocks: int, qtype: int):
    """Upload raw Q4_K / Q6_K bytes once (qk_cuda.py:252-270); raises CudaRegistrationError on failure."""
    lib = _dev()
    if lib is None:
        return None
    _require_weight_bytes(weight_raw, out_f, n_blocks, qtype)
    w = _raw(weight_raw)
    with _LOCK:
        h = lib.qk_register_weight(w.ctypes.data, int(out_f), int(n_blocks), int(qtype))
    if h < 0:
        raise CudaRegistrationError(f"resident weight registration failed for [{out_f}, {n_blocks * 256}] (qtype={qtype})")
    return int(h)


def apply_resident(handle: int, x_int: np.ndarray, out_f: int, fw: int):
    lib = _dev()
    if lib is None:
        return None
    x = np.ascontiguousarray(np.atleast_2d(np.asarray(x_int, dtype=np.int64)))
    out = np.empty((x.shape[0], out_f), dtype=np.int64)
    with _LOCK:
        rc = lib.qk_apply_resident(int(handle), x.ctypes.data, x.shape[0], int(fw), out.ctypes.data)
    return None if rc != 0 else out


def grouped_available() -> bool:
    return available()


def apply_resident_grouped(handles, x_int: np.ndarray, out_features, fw: int, phase_ids=None):
    """Same-input resident projections with one upload and one download (qk_cuda.py:405-442)."""
    lib = _dev()
    if lib is None:
        return None
    hs = tuple(int(h) for h in handles)
    ofs = tuple(int(n) for n in out_features)
    if not hs or len(hs) != len(ofs) or len(hs) > 16 or any(n <= 0 for n in ofs):
        raise ValueError("grouped resident apply requires 1..16 handles and matching positive output sizes")
    phases = tuple(0 for _ in hs) if phase_ids is None else tuple(int(p) for p in phase_ids)
    if len(phases) != len(hs) or any(p not in (0, 1, 2, 3, 4) for p in phases):
        raise ValueError("grouped resident phase_ids must match handles and use known Q/K/V/O identifiers")
    x = np.ascontiguousarray(np.atleast_2d(np.asarray(x_int, dtype=np.int64)))
    rows = int(x.shape[0])
    total = rows * sum(ofs)
    flat = np.empty(total, dtype=np.int64)
    harr = (ctypes.c_int64 * len(hs))(*hs)
    parr = (ctypes.c_int * len(phases))(*phases)
    with _LOCK:
        rc = lib.qk_apply_resident_grouped(harr, parr, len(hs), x.ctypes.data, rows, int(fw), total, flat.ctypes.data)
    if rc != 0:
        return None
    result, offset = [], 0
    for out_f in ofs:
        result.append(flat[offset:offset + rows * out_f].reshape(rows, out_f))
        offset += rows * out_f
    return tuple(result)


def _balanced_capacity(L: int) -> int:
    return 127 * ((256 ** L - 1) // 255)


def limbs_needed(maxabs: int) -> int:
    """Smallest balanced base-256 digit count representing +-|x| exactly (qk_cuda.py:979-992)."""
    m = int(maxabs)
    L = 1
    while L < 8 and m > _balanced_capacity(L):
        L += 1
    if m > _balanced_capacity(8):
        raise OverflowError(f"|x| max {m} exceeds 8 balanced base-256 digits ({_balanced_capacity(8)})")
    return L


def dp4a_available() -> bool:
    return available()


def apply_resident_dp4a(handle: int, x_int: np.ndarray, out_f: int, fw: int, qtype: int, ln: int = None):
    """Limb-decomposed apply (qk_cuda.py:1029-1046). The gfx950 kernel is exact for every activation, so the
    result is ``apply_resident``'s; argument checks follow the reference."""
    if qtype not in (Q4_K, Q6_K):
        raise ValueError(f"unknown qtype {qtype} (expected Q4_K={Q4_K} or Q6_K={Q6_K})")
    lib = _dev()
    if lib is None:
        return None
    x = np.ascontiguousarray(np.atleast_2d(np.asarray(x_int, dtype=np.int64)))
    if ln is not None:
        need = limbs_needed(max(abs(int(x.min())), abs(int(x.max()))) if x.size else 0)
        if not 1 <= int(ln) <= 4 or int(ln) < need:
            raise ValueError(f"DP4A limb count {ln} invalid for activations needing {need}")
    fn = lib.qk_apply_resident_q4k_dp4a if qtype == Q4_K else lib.qk_apply_resident_q6k_dp4a
    out = np.empty((x.shape[0], out_f), dtype=np.int64)
    with _LOCK:
        rc = fn(int(handle), x.ctypes.data, x.shape[0], int(fw), int(ln or 4), out.ctypes.data)
    return None if rc != 0 else out


def moe_ffn_available() -> bool:
    return available()


def moe_ffn_batched_available() -> bool:
    return available()


def moe_ffn_batched(gate_h, up_h, down_h, m: int, k: int, h, gates, d_model: int, e_ffn: int, fa: int, fw: int,
                    *, dp4a: bool = False):
    """Batched MoE over all m*k (token, expert) pairs (qk_cuda.py:1073-1101); pairs flattened token-major."""
    lib = _dev()
    if lib is None:
        return None
    P = m * k
    if m <= 0 or k <= 0:
        raise ValueError(f"batched MoE requires positive m and k, got m={m}, k={k}")
    if len(gate_h) != P or len(up_h) != P or len(down_h) != P:
        raise ValueError(f"batched MoE requires exactly m*k={P} handles for each projection")
    arr = lambda hs: (ctypes.c_int64 * P)(*[int(v) for v in hs])
    hh = np.ascontiguousarray(np.asarray(h, np.int64).reshape(-1))
    gg = np.ascontiguousarray(np.asarray(gates, np.int64).reshape(-1))
    if hh.size != m * d_model or gg.size != P:
        raise ValueError(f"batched MoE expected h.size={m * d_model} and gates.size={P}, got {hh.size} and {gg.size}")
    out = np.empty((m, d_model), dtype=np.int64)
    fn = lib.qk_moe_ffn_batched_dp4a if dp4a else lib.qk_moe_ffn_batched
    with _LOCK:
        rc = fn(arr(gate_h), arr(up_h), arr(down_h), int(m), int(k), hh.ctypes.data, gg.ctypes.data, int(d_model),
                int(e_ffn), int(fa), int(fw), out.ctypes.data)
    return None if rc != 0 else out


def moe_ffn(gate_h, up_h, down_h, h, gates, d_model: int, e_ffn: int, fa: int, fw: int, dp4a: bool = False):
    """One token's MoE FFN over its selected experts (qk_cuda.py:1104-1124)."""
    n_e = len(gate_h)
    if n_e <= 0 or len(up_h) != n_e or len(down_h) != n_e:
        raise ValueError("MoE requires the same positive number of gate, up, and down handles")
    out = moe_ffn_batched(gate_h, up_h, down_h, 1, n_e, h, gates, d_model, e_ffn, fa, fw, dp4a=dp4a)
    return None if out is None else out[0]


def free_all() -> None:
    lib = _dev()
    if lib is not None:
        with _LOCK:
            lib.qk_free_all()


def resident_count() -> int:
    lib = _dev()
    return 0 if lib is None else int(lib.qk_resident_count())


def resident_capacity() -> int:
    lib = _dev()
    return 0 if lib is None else int(lib.qk_resident_capacity())


def reserve_resident_capacity(count: int) -> bool:
    if int(count) < 0:
        raise ValueError("resident capacity must be non-negative")
    lib = _dev()
    return lib is not None and lib.qk_resident_reserve(int(count)) == 0


def moe_workspace_bytes() -> "int | None":
    lib = _dev()
    return None if lib is None else int(lib.qk_moe_workspace_bytes())


def release_moe_workspace() -> bool:
    lib = _dev()
    if lib is None:
        return False
    lib.qk_moe_workspace_release()
    return True
