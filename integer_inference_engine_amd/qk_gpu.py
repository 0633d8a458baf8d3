"""gfx950 producer boundary for the north-mini-code Q4_K / Q6_K hot path.

Mirrors ``north-mini-code/src/nmc/qk_cuda.py`` (functions ``available``, ``qk_linear``, ``register_weight``,
``apply_resident``, ``apply_resident_grouped``, ``apply_resident_dp4a``, ``moe_ffn``, ``moe_ffn_batched``,
``free_all``, ``resident_count``, ``limbs_needed`` ...; qk_cuda.py:226-1124) with the same arguments and return
conventions: ``None`` on a library rc != 0, ``CudaRegistrationError`` when a registration fails. Calls are
serialized by a process lock as in the reference (qk_cuda.py:35-38).
"""
from __future__ import annotations

import contextlib
import ctypes
import threading
from dataclasses import dataclass

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


# ---- resident preprocessing and attention bank (qk_cuda.py:285-715) -----------------------------------------
class CudaContextError(RuntimeError):
    """A resident request context failed validation, allocation, or an exact envelope guard (qk_cuda.py:79-80)."""


def register_i64(weight_int, rows: int = None, cols: int = None) -> int:
    """Upload a dense int64 matrix (norm gain [1, d] or router [experts, d]); handle or CudaRegistrationError."""
    lib = _dev()
    if lib is None:
        raise CudaRegistrationError("gfx950 device unavailable")
    w = np.ascontiguousarray(np.atleast_2d(np.asarray(weight_int, dtype=np.int64)))
    r, c = w.shape if rows is None else (int(rows), int(cols))
    if w.size != r * c or r <= 0 or c <= 0:
        raise ValueError("int64 registration shape does not match the data")
    with _LOCK:
        h = int(lib.qk_register_i64(w.ctypes.data, r, c))
    if h < 0:
        raise CudaRegistrationError(f"resident int64 registration failed for shape [{r}, {c}]")
    return h


def _rms_envelope_ok(x: np.ndarray) -> bool:
    """Every row's sum of squares fits signed 128 bits (the producer's exact RMSNorm envelope)."""
    lim = (1 << 127) - 1
    for row in x:
        m = max(abs(int(row.min())), abs(int(row.max())))
        if m * m * x.shape[1] <= lim:
            continue
        if sum(int(v) * int(v) for v in row) > lim:
            return False
    return True


def rmsnorm_router(gain_handle: int, router_handle: int, x_int, n_used: int, fa: int, fw: int, eps: int = 1):
    """(normalized h [T, D], selected ids [T, K] int32, gates [T, K]) or None outside the envelope (the caller's
    host path then runs); shape or runtime failures raise (qk_cuda.py:331-372)."""
    lib = _dev()
    if lib is None:
        return None
    x = np.asarray(x_int, dtype=np.int64)
    x = x.reshape(1, -1) if x.ndim == 1 else x
    if x.ndim != 2 or x.shape[0] <= 0 or x.shape[1] <= 0:
        raise ValueError("resident RMSNorm/router requires a non-empty vector or 2-D activation")
    n_used, fa, fw, eps = int(n_used), int(fa), int(fw), int(eps)
    if not 0 < n_used <= np.iinfo(np.int32).max or not 1 <= fa <= 29 or not 0 <= fw <= 62 or \
            not 0 <= eps < (1 << 64):
        raise ValueError("resident RMSNorm/router parameters are outside the native envelope")
    x = np.ascontiguousarray(x)
    if not _rms_envelope_ok(x):
        return None
    rows = x.shape[0]
    h = np.empty_like(x)
    ids = np.empty((rows, n_used), dtype=np.int32)
    gates = np.empty((rows, n_used), dtype=np.int64)
    with _LOCK:
        rc = int(lib.qk_rmsnorm_router(int(gain_handle), int(router_handle), x.ctypes.data, rows, fa, fw, eps, n_used,
                                       h.size, ids.size, h.ctypes.data, ids.ctypes.data, gates.ctypes.data))
    if rc == 3:
        return None
    if rc != 0:
        raise CudaContextError(f"resident RMSNorm/router failed with native status {rc}")
    return h, ids, gates


def resident_attention_available() -> bool:
    return _dev() is not None


def resident_layer_available() -> bool:
    return _dev() is not None


class ResidentLayerHidden:
    """Marker for the M=1 residual a bank retains between MoE layers (no host activation). It is valid only for
    the bank and the bank epoch that produced it."""

    __slots__ = ("_cache", "_generation", "shape")

    def __init__(self, cache, generation: int):
        self._cache, self._generation = cache, int(generation)
        self.shape = (1, cache.d_model)


@dataclass
class _BankLayer:
    """Host-side view of one bank layer: tokens held on the device and the MoE shape it was configured with."""
    length: int = 0
    moe: "tuple | None" = None          # (n_experts, n_used, d_model, expert_ffn)


def _why(rc: int, *, cold_rc: bool = False) -> str:
    """Caller-facing reason for a nonzero bank status."""
    if rc == 3:
        return "exact overflow guard fired"
    if cold_rc and rc == 4:
        return "selected cold experts remain unbound"
    return f"native status {rc}"


class ResidentAttentionCache:
    """Request-scoped device K/V bank with the exact M=1 attention sublayer and the MoE layer begin / continue
    chain (interface: qk_cuda.py:476-715; native side: ``qk_attention_bank_*``). A failed native call poisons
    the layer on the device and raises CudaContextError.

    State kept here: one ``_BankLayer`` per layer, the layer whose MoE half is open between ``begin`` and
    ``continue`` (at most one), and an epoch that every reset / continuation / close advances so that stale
    ``ResidentLayerHidden`` markers are rejected."""

    def __init__(self, n_layers: int, max_length: int, d_model: int, n_heads: int, n_kv: int, head_dim: int,
                 fa: int, cos, sin):
        lib = _dev()
        if lib is None:
            raise CudaContextError("resident attention context API is unavailable")
        dims = tuple(int(v) for v in (n_layers, max_length, d_model, n_heads, n_kv, head_dim, fa))
        n_layers, max_length, d_model, n_heads, n_kv, head_dim, fa = dims
        shape_ok = min(dims[:6]) > 0 and n_heads % n_kv == 0 and head_dim % 2 == 0
        native_ok = 1 <= fa <= 29 and d_model % 256 == 0 and (n_heads * head_dim) % 256 == 0
        if not (shape_ok and native_ok):
            raise ValueError("invalid resident attention dimensions")
        tables = [np.ascontiguousarray(np.asarray(t, dtype=np.int64)) for t in (cos, sin)]
        if any(t.shape != (max_length, head_dim // 2) for t in tables):
            raise ValueError(f"resident attention RoPE tables must both have shape {(max_length, head_dim // 2)}")
        with _LOCK:
            self.handle = int(lib.qk_attention_bank_create(*dims, tables[0].ctypes.data, tables[1].ctypes.data))
        if self.handle < 0:
            raise CudaContextError("resident attention context creation failed")
        self.n_layers, self.max_length, self.d_model = n_layers, max_length, d_model
        self.n_heads, self.n_kv, self.head_dim, self.fa = n_heads, n_kv, head_dim, fa
        self.q_width = n_heads * head_dim
        self.inv_sqrt = int(round((1 << fa) / float(np.sqrt(head_dim))))
        self._layers = [_BankLayer() for _ in range(n_layers)]
        self._open_layer = None
        self._epoch = 0
        self._closed = False

    # -- helpers ---------------------------------------------------------------------------------------------------
    def _native(self, fn: str, *args) -> int:
        """Call ``qk_attention_bank_<fn>(handle, *args)`` under the process lock; the open check comes first."""
        if self._closed:
            raise CudaContextError("resident attention context is closed")
        with _LOCK:
            rc = getattr(_lib.lib(), "qk_attention_bank_" + fn)(self.handle, *args)
        return 0 if rc is None else int(rc)

    def _layer(self, layer) -> "_BankLayer | None":
        layer = int(layer)
        return self._layers[layer] if 0 <= layer < self.n_layers else None

    def _row(self, hidden, what: str) -> np.ndarray:
        x = np.ascontiguousarray(np.asarray(hidden, dtype=np.int64))
        if x.shape != (1, self.d_model):
            raise ValueError(f"resident {what} expects hidden shape (1, {self.d_model})")
        return x

    def _room(self, layer) -> bool:
        st = self._layer(layer)
        return st is not None and st.length < self.max_length

    @property
    def _generation(self) -> int:
        return self._epoch

    def length(self, layer=0):
        return self._layers[layer].length

    # -- K/V and the attention sublayer ----------------------------------------------------------------------------
    def import_layer(self, layer: int, k, v) -> None:
        kk, vv = (np.ascontiguousarray(np.asarray(t, dtype=np.int64)) for t in (k, v))
        if kk.shape != vv.shape or kk.ndim != 3 or kk.shape[0] != self.n_kv or kk.shape[2] != self.head_dim:
            raise ValueError("resident attention import expects matching [n_kv, length, head_dim] K/V")
        st = self._layer(layer)
        if st is None or kk.shape[1] > self.max_length:
            raise ValueError("resident attention import exceeds layer or context bounds")
        if self._native("import", int(layer), kk.ctypes.data, vv.ctypes.data, kk.shape[1]) != 0:
            raise CudaContextError(f"resident attention K/V import failed for layer {layer}")
        st.length = int(kk.shape[1])

    def apply(self, layer: int, q_handle: int, k_handle: int, v_handle: int, o_handle: int, hidden, fw: int,
              window, rope: bool):
        if not self._room(layer):
            raise ValueError("resident attention decode exceeds layer or context bounds")
        x = self._row(hidden, "attention apply")
        out = np.empty_like(x)
        rc = self._native("apply", int(layer), int(q_handle), int(k_handle), int(v_handle), int(o_handle),
                          x.ctypes.data, int(fw), -1 if window is None else int(window), int(bool(rope)),
                          self.inv_sqrt, out.size, out.ctypes.data)
        if rc != 0:
            raise CudaContextError(f"resident attention apply failed for layer {layer}: {_why(rc)}")
        self._layers[int(layer)].length += 1
        return out

    # -- MoE layers ------------------------------------------------------------------------------------------------
    def configure_moe_layer(self, layer: int, n_experts: int, n_used: int, d_model: int, expert_ffn: int) -> None:
        shape = tuple(int(v) for v in (n_experts, n_used, d_model, expert_ffn))
        n_exp, used, width, ffn = shape
        st = self._layer(layer)
        if st is None or not (0 < used <= n_exp) or width != self.d_model or width % 256 or ffn <= 0 or ffn % 256:
            raise ValueError("invalid resident MoE layer dimensions")
        if st.moe not in (None, shape):
            raise ValueError("resident MoE layer cannot be reconfigured with different dimensions")
        if self._native("moe_configure", int(layer), *shape) != 0:
            raise CudaContextError(f"resident MoE layer configuration failed for layer {layer}")
        st.moe = shape

    def bind_moe_expert(self, layer: int, expert: int, gate_handle: int, up_handle: int, down_handle: int) -> None:
        st = self._layer(layer)
        if st is None or st.moe is None or not 0 <= int(expert) < st.moe[0]:
            raise ValueError("resident MoE expert binding is outside the configured layer")
        if self._native("moe_bind", int(layer), int(expert), int(gate_handle), int(up_handle), int(down_handle)):
            raise CudaContextError(f"resident MoE expert binding failed for layer {layer}, expert {expert}")

    def begin_moe_layer(self, layer: int, gain_handle: int, router_handle: int, q_handle: int, k_handle: int,
                        v_handle: int, o_handle: int, hidden, fw: int, eps: int, window, rope: bool) -> tuple:
        st = self._layer(layer)
        if st is None or st.moe is None or self._open_layer is not None or st.length >= self.max_length:
            raise ValueError("resident MoE layer begin violates configuration, pending, or context bounds")
        if isinstance(hidden, ResidentLayerHidden):
            if hidden._cache is not self or hidden._generation != self._epoch:
                raise ValueError("resident hidden marker is stale or belongs to another request")
            x_ptr, retained = None, 1
        else:
            x = self._row(hidden, "MoE layer begin")
            x_ptr, retained = x.ctypes.data, 0
        cold = np.empty(st.moe[1], dtype=np.int32)
        n_cold = ctypes.c_int(0)
        rc = self._native("moe_begin", int(layer), int(gain_handle), int(router_handle), int(q_handle),
                          int(k_handle), int(v_handle), int(o_handle), x_ptr, retained, int(fw), int(eps),
                          -1 if window is None else int(window), int(bool(rope)), self.inv_sqrt, cold.size,
                          ctypes.byref(n_cold), cold.ctypes.data)
        if rc != 0:
            raise CudaContextError(f"resident MoE layer begin failed for layer {layer}: {_why(rc)}")
        if not 0 <= n_cold.value <= cold.size:
            raise CudaContextError("resident MoE layer returned an invalid cold-route count")
        st.length += 1
        self._open_layer = int(layer)
        return tuple(cold[:n_cold.value].tolist())

    def continue_moe_layer(self, layer: int, fw: int, *, publish: bool = False):
        if self._open_layer is None or self._open_layer != int(layer):
            raise ValueError("resident MoE continuation has no matching prepared layer")
        out = np.empty((1, self.d_model), dtype=np.int64) if publish else None
        rc = self._native("moe_continue", int(layer), int(fw), int(bool(publish)),
                          0 if out is None else out.size, None if out is None else out.ctypes.data)
        if rc != 0:
            raise CudaContextError(f"resident MoE continuation failed for layer {layer}: {_why(rc, cold_rc=True)}")
        self._open_layer = None
        self._epoch += 1
        return out if publish else ResidentLayerHidden(self, self._epoch)

    def export_moe_hidden(self) -> np.ndarray:
        if self._open_layer is not None:
            raise CudaContextError("resident MoE hidden cannot be exported from this context state")
        out = np.empty((1, self.d_model), dtype=np.int64)
        if self._native("moe_export", out.size, out.ctypes.data) != 0:
            raise CudaContextError("resident MoE hidden export failed")
        return out

    # -- lifetime --------------------------------------------------------------------------------------------------
    def workspace_bytes(self) -> int:
        v = self._native("workspace_bytes")
        if v == (1 << 64) - 1:
            raise CudaContextError("resident attention workspace accounting failed")
        return v

    def reset(self) -> None:
        if self._native("reset") != 0:
            raise CudaContextError("resident attention context reset failed")
        for st in self._layers:
            st.length = 0
        self._open_layer = None
        self._epoch += 1

    def close(self) -> None:
        if self._closed:
            return
        self._native("destroy")
        self._closed = True
        self._open_layer = None
        self._epoch += 1


# ---- telemetry and capability probes (qk_cuda.py:24-34, 870-910, 1029-1101) ---------------------------------------
PROFILE_METRICS = (
    "registration_calls", "registration_ns",
    "h2d_calls", "h2d_bytes", "h2d_ns",
    "d2h_calls", "d2h_bytes", "d2h_ns",
    "allocation_calls", "allocation_bytes", "allocation_ns", "free_calls",
    "native_calls", "resident_apply_calls", "grouped_apply_calls",
    "moe_calls", "moe_batched_calls", "moe_batched_dp4a_calls",
    "q_projection_calls", "q_projection_ns", "k_projection_calls", "k_projection_ns",
    "v_projection_calls", "v_projection_ns", "o_projection_calls", "o_projection_ns",
    "other_projection_calls", "other_projection_ns",
)


def resident_preprocess_available() -> bool:
    """Whether the exact resident RMSNorm / router / top-k boundary is usable (qk_cuda.py:319-322)."""
    lib = _dev()
    return lib is not None and hasattr(lib, "qk_register_i64") and hasattr(lib, "qk_rmsnorm_router")


def resident_preprocess_bytes(n_layers: int, d_model: int, n_experts: int) -> int:
    """Device bytes of the per-layer int64 norm gains plus router matrices (expert slices excluded: they are
    registered lazily by route)."""
    n_layers, d_model, n_experts = int(n_layers), int(d_model), int(n_experts)
    if n_layers < 0 or d_model <= 0 or n_experts <= 0:
        raise ValueError("resident preprocessing memory dimensions must be non-negative layers and positive widths")
    return n_layers * (n_experts + 1) * d_model * np.dtype(np.int64).itemsize


def profile_reset(*, enabled: bool = True) -> bool:
    """Zero the boundary counters and enable / disable them."""
    lib = _dev()
    if lib is None:
        return False
    with _LOCK:
        lib.qk_profile_set_enabled(0)
        lib.qk_profile_reset()
        lib.qk_profile_set_enabled(int(bool(enabled)))
    return True


def profile_set_enabled(enabled: bool) -> bool:
    lib = _dev()
    if lib is None:
        return False
    with _LOCK:
        lib.qk_profile_set_enabled(int(bool(enabled)))
    return True


def profile_snapshot() -> "dict | None":
    """Allocation / copy / call counters of the current profile window, by name."""
    import ctypes
    lib = _dev()
    if lib is None:
        return None
    values = (ctypes.c_uint64 * len(PROFILE_METRICS))()
    with _LOCK:
        required = int(lib.qk_profile_snapshot(values, len(values)))
    if required != len(PROFILE_METRICS):
        raise RuntimeError(f"profile metric ABI mismatch: native={required}, python={len(PROFILE_METRICS)}")
    return {name: int(values[i]) for i, name in enumerate(PROFILE_METRICS)}


def moe_workspace_allocations() -> "int | None":
    """Number of MoE workspace grows since free_all."""
    lib = _dev()
    if lib is None:
        return None
    with _LOCK:
        return int(lib.qk_moe_workspace_allocations())


def apply_resident_q6k_dp4a(handle: int, x_int: np.ndarray, out_f: int, fw: int, ln: int = None):
    return apply_resident_dp4a(handle, x_int, out_f, fw, 1, ln)


def moe_ffn_dp4a_available() -> bool:
    lib = _dev()
    return lib is not None and hasattr(lib, "qk_moe_ffn_dp4a")


def moe_ffn_batched_dp4a_available() -> bool:
    lib = _dev()
    return lib is not None and hasattr(lib, "qk_moe_ffn_batched_dp4a")


# ---- retained MoE token chain (qk_cuda.py:726-868) ------------------------------------------------------------------
@dataclass(frozen=True)
class ResidentMoeLayerSpec:
    """Resident dense-handle inputs of one M = 1 MoE layer."""
    layer: int
    gain_handle: int
    router_handle: int
    q_handle: int
    k_handle: int
    v_handle: int
    o_handle: int
    window: "int | None"
    rope: bool


def _expert_handles(value, where: str):
    """A (gate, up, down) triple of non-negative resident handles, or CudaContextError naming ``where``."""
    try:
        triple = tuple(int(h) for h in value)
    except (TypeError, ValueError):
        triple = None
    if triple is None or len(triple) != 3 or min(triple) < 0:
        raise CudaContextError(f"{where} did not return a valid gate/up/down handle triplet")
    return triple


class ResidentMoeTokenExecutor:
    """One token through consecutive MoE layers of a ResidentAttentionCache with the hidden state retained on the
    device between layers (interface: qk_cuda.py:726-868, used by engine.py's resident decode).

    ``lookup_expert(layer, e)`` returns an already resident (gate, up, down) triplet or None, with no side
    effects; ``load_expert(layer, e)`` is called only for the experts the device reports unbound after routing.
    Any error raised while touching the bank poisons the executor: the caller resets or destroys the bank instead
    of mixing partly advanced K/V with another path.

    Per layer the executor keeps one entry in ``_ready``: the set of experts bound to the bank for that layer. A
    layer gets its entry once it is configured and every expert ``lookup_expert`` knows has been bound."""

    def __init__(self, cache: "ResidentAttentionCache", *, first_layer: int, layer_count: int, n_experts: int,
                 n_used: int, d_model: int, expert_ffn: int, fw: int, eps: int, lookup_expert, load_expert):
        if not isinstance(cache, ResidentAttentionCache) or cache._closed:
            raise ValueError("resident token executor requires an open attention bank")
        first_layer, layer_count, n_experts, n_used, d_model, expert_ffn, fw, eps = map(
            int, (first_layer, layer_count, n_experts, n_used, d_model, expert_ffn, fw, eps))
        layers_ok = first_layer >= 0 and layer_count > 0 and first_layer + layer_count <= cache.n_layers
        moe_ok = n_experts > 0 and 0 < n_used <= n_experts and expert_ffn > 0 and expert_ffn % 256 == 0
        width_ok = d_model == cache.d_model and d_model % 256 == 0
        fixed_ok = 0 <= fw <= 62 and 0 <= eps < (1 << 64)
        if not (layers_ok and moe_ok and width_ok and fixed_ok):
            raise ValueError("invalid resident token executor dimensions")
        if not (callable(lookup_expert) and callable(load_expert)):
            raise TypeError("resident token executor requires expert lookup and lazy-load callables")
        self.cache = cache
        self.first_layer, self.layer_count = first_layer, layer_count
        self.n_experts, self.n_used, self.d_model, self.expert_ffn = n_experts, n_used, d_model, expert_ffn
        self.fw, self.eps = fw, eps
        self.lookup_expert, self.load_expert = lookup_expert, load_expert
        self._ready: "dict[int, set[int]]" = {}
        self._poisoned = False

    @property
    def poisoned(self) -> bool:
        return self._poisoned

    @contextlib.contextmanager
    def _guarded(self):
        """Refuse work once poisoned; poison on any exception raised inside."""
        if self._poisoned:
            raise CudaContextError("resident token executor is poisoned; destroy or reset the request bank")
        try:
            yield
        except BaseException:
            self._poisoned = True
            raise

    def _check_specs(self, layers) -> "list[ResidentMoeLayerSpec]":
        specs = list(layers)
        last = self.first_layer + self.layer_count - 1
        good = len(specs) == self.layer_count and all(
            isinstance(s, ResidentMoeLayerSpec) and int(s.layer) == self.first_layer + i for i, s in enumerate(specs))
        if not good:
            raise ValueError(f"resident token executor requires consecutive layers {self.first_layer}..{last}")
        return specs

    def _bind(self, layer: int, expert: int, triple) -> None:
        self.cache.bind_moe_expert(layer, expert, *triple)
        self._ready[layer].add(expert)

    def _make_ready(self, layer: int) -> None:
        if layer in self._ready:
            return
        self.cache.configure_moe_layer(layer, self.n_experts, self.n_used, self.d_model, self.expert_ffn)
        self._ready[layer] = set()
        for expert in range(self.n_experts):
            found = self.lookup_expert(layer, expert)
            if found is not None:
                where = f"resident expert lookup for layer {layer}, expert {expert}"
                self._bind(layer, expert, _expert_handles(found, where))

    def prepare(self, layers):
        """Configure every layer and bind the experts already resident, before any K/V changes."""
        if self._poisoned:
            raise CudaContextError("resident token executor is poisoned; destroy or reset the request bank")
        specs = self._check_specs(layers)
        with self._guarded():
            for spec in specs:
                self._make_ready(int(spec.layer))
        return tuple(specs)

    def run(self, hidden, layers) -> np.ndarray:
        specs = self.prepare(layers)
        state = np.ascontiguousarray(np.asarray(hidden, dtype=np.int64))
        if state.shape != (1, self.d_model):
            raise ValueError(f"resident token executor expects hidden shape (1, {self.d_model})")
        with self._guarded():
            for spec in specs:
                layer = int(spec.layer)
                cold = self.cache.begin_moe_layer(
                    layer, int(spec.gain_handle), int(spec.router_handle), int(spec.q_handle), int(spec.k_handle),
                    int(spec.v_handle), int(spec.o_handle), state, self.fw, self.eps, spec.window, bool(spec.rope))
                if len(set(cold)) != len(cold) or not all(0 <= e < self.n_experts for e in cold):
                    raise CudaContextError(f"resident layer {layer} returned invalid cold expert IDs")
                for expert in cold:
                    where = f"lazy expert loader for layer {layer}, expert {expert}"
                    self._bind(layer, expert, _expert_handles(self.load_expert(layer, expert), where))
                state = self.cache.continue_moe_layer(layer, self.fw, publish=spec is specs[-1])
            if not (isinstance(state, np.ndarray) and state.shape == (1, self.d_model)):
                raise CudaContextError("resident token executor did not publish its final residual")
        return state
