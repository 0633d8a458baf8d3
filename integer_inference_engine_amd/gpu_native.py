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
    """Limb-decomposed Q1 apply through ``bonsai_q1_linear_dp4a_gpu`` (gpu_native.py:226-261): L = 4 when the
    activations fit the balanced base-256 L=4 range, else 8; an explicit L=4 outside it raises; rc != 0 (the
    library's own L=4 guard included) gives None."""
    lib = _dev()
    if lib is None:
        return None
    x = _as_i64_2d(x_fp)
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint8))
    s = np.ascontiguousarray(np.asarray(scale_fp, dtype=np.int64))
    out_f, n_blocks = s.shape
    if x.shape[1] != n_blocks * 128:
        raise ValueError(f"Q1_0 contraction mismatch: x has {x.shape[1]}, weight expects {n_blocks * 128}")
    if L is None:
        mn, mx = (int(x.min()), int(x.max())) if x.size else (0, 0)
        L = 4 if (_L4_LO <= mn and mx <= _L4_HI) else 8
    elif int(L) == 4 and x.size:
        mn, mx = int(x.min()), int(x.max())
        if not (_L4_LO <= mn and mx <= _L4_HI):
            raise ValueError(f"q1_apply_dp4a_gpu: explicit L=4 requires activations in [{_L4_LO}, {_L4_HI}], "
                             f"got [{mn}, {mx}]; use L=8 (always exact) or L=None")
    out = np.empty((x.shape[0], out_f), dtype=np.int64)
    rc = lib.bonsai_q1_linear_dp4a_gpu(x.ctypes.data, b.ctypes.data, s.ctypes.data, x.shape[0], int(out_f),
                                       int(n_blocks), int(frac), int(L), out.ctypes.data)
    return None if rc != 0 else out


def residency_available() -> bool:
    return _dev() is not None


def q1_register_weight(bits: np.ndarray, scale_fp: np.ndarray, *, gpu_coalesced: bool = False,
                       gpu_bmma: bool = False) -> "int | None":
    """Upload bits + scale once; return a handle >= 0 or None (gpu_native.py:270-306). The weight is stored in
    the gfx950 tile layout; scales are narrowed to int32 on device when lossless. ``gpu_coalesced`` /
    ``gpu_bmma`` bind the reference's layout-specific entry points (same refusals: int32 scales only, and
    out_features % 8 == 0 for bmma); on gfx950 all three store the same tile layout."""
    lib = _dev()
    if lib is None:
        return None
    if gpu_coalesced and gpu_bmma:
        raise ValueError("choose one GPU Q1 runtime layout")
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint8))
    src = np.asarray(scale_fp)
    if not np.issubdtype(src.dtype, np.integer):
        raise TypeError(f"Q1_0 scale must be an integer dtype, got {src.dtype}")
    use_i32 = src.dtype.itemsize <= 4
    if (gpu_coalesced or gpu_bmma) and not use_i32:
        raise ValueError("GPU-coalesced Q1 registration currently requires committed int32 scales")
    if use_i32:
        s = np.ascontiguousarray(src, dtype=np.int32)
        fn = (lib.bonsai_q1_register_weight_i32_bmma if gpu_bmma else
              lib.bonsai_q1_register_weight_i32_gpu_layout if gpu_coalesced else lib.bonsai_q1_register_weight_i32)
        h = fn(b.ctypes.data, s.ctypes.data, int(s.shape[0]), int(s.shape[1]))
    else:
        s = np.ascontiguousarray(src, dtype=np.int64)
        h = lib.bonsai_q1_register_weight(b.ctypes.data, s.ctypes.data, int(s.shape[0]), int(s.shape[1]))
    return None if int(h) < 0 else int(h)


def gpu_reservation_create(component_bytes) -> "tuple[int, int] | None":
    """Reserve several exact device allocations as one failure-atomic probe (gpu_native.py:334-355): (handle,
    allocated_bytes), or None with nothing left allocated."""
    lib = _dev()
    if lib is None:
        return None
    sizes = np.ascontiguousarray(np.asarray(tuple(component_bytes), dtype=np.uint64))
    if sizes.ndim != 1 or sizes.size == 0 or np.any(sizes == 0):
        raise ValueError("GPU reservation components must be a non-empty list of positive byte counts")
    allocated = ctypes.c_uint64()
    h = lib.bonsai_gpu_reservation_create(sizes.ctypes.data, int(sizes.size), ctypes.byref(allocated))
    return None if int(h) < 0 else (int(h), int(allocated.value))


def gpu_reservation_free(handle: int) -> None:
    """Release a reservation; safe to call more than once."""
    lib = _dev()
    if lib is not None:
        lib.bonsai_gpu_reservation_free(int(handle))


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


def rmsnorm_gpu(x_fp: np.ndarray, frac: int, eps: int = 1, gain_q: "np.ndarray | None" = None) -> "np.ndarray | None":
    """Integer RMSNorm (gpu_native.py:390-415); None on rc 4 (128-bit or gain envelope)."""
    lib = _dev()
    if lib is None:
        return None
    x = _as_i64_2d(x_fp)
    rows, cols = x.shape
    out = np.empty((rows, cols), dtype=np.int64)
    g = None
    if gain_q is not None:
        g = np.ascontiguousarray(np.asarray(gain_q, dtype=np.int64))
        if g.shape[0] != cols:
            raise ValueError(f"RMSNorm gain has {g.shape[0]} elems, expected cols={cols}")
    rc = lib.bonsai_rmsnorm_gpu(x.ctypes.data, rows, cols, int(frac), int(eps), None if g is None else g.ctypes.data,
                                out.ctypes.data)
    return None if rc != 0 else out


def silu_gpu(x_fp: np.ndarray, frac: int) -> "np.ndarray | None":
    """Bonsai SiLU ``(x * sigmoid(x)) >> frac`` with mod-2^64 wrap (q1_native.py:1895 ``silu_native``)."""
    lib = _dev()
    if lib is None:
        return None
    x = np.ascontiguousarray(np.asarray(x_fp, dtype=np.int64))
    out = np.empty_like(x)
    rc = lib.bonsai_silu_gpu(x.ctypes.data, x.size, int(frac), out.ctypes.data)
    return None if rc != 0 else out


def rope_neox_gpu(x_fp: np.ndarray, positions, cos: np.ndarray, sin: np.ndarray, frac: int) -> "np.ndarray | None":
    """NeoX RoPE (rope_v2.py:92-117) of x (rows, nh, hd), row r at table row positions[r]; None where the oracle
    raises on the int64 envelope."""
    lib = _dev()
    if lib is None:
        return None
    x = np.ascontiguousarray(np.asarray(x_fp, dtype=np.int64))
    rows, nh, hd = x.shape
    pos = np.ascontiguousarray(np.asarray(positions, dtype=np.int64))
    c = np.ascontiguousarray(np.asarray(cos, dtype=np.int64))
    s = np.ascontiguousarray(np.asarray(sin, dtype=np.int64))
    out = np.empty_like(x)
    rc = lib.imie_rope_neox_gpu(x.ctypes.data, rows, nh, hd, pos.ctypes.data, c.ctypes.data, s.ctypes.data,
                                c.shape[0], int(frac), out.ctypes.data)
    return None if rc != 0 else out


def argmax_gpu(logits: np.ndarray) -> "np.ndarray | None":
    """Row argmax with the lowest index on ties (reference_bonsai.py:812-827)."""
    lib = _dev()
    if lib is None:
        return None
    z = _as_i64_2d(logits)
    ids = np.empty(z.shape[0], dtype=np.int64)
    rc = lib.imie_argmax_gpu(z.ctypes.data, z.shape[0], z.shape[1], ids.ctypes.data)
    return None if rc != 0 else ids


def attention_prefill_gpu(q_fp, k_fp, v_fp, start: int, frac: int, inv_sqrt_fp: int) -> "np.ndarray | None":
    """Causal attention (gpu_native.py:418-446): q (H, M, hd) post q-norm + RoPE, k/v (Hkv, L, hd), L = start + M.
    None on an envelope overflow (rc 2)."""
    lib = _dev()
    if lib is None:
        return None
    q = np.ascontiguousarray(q_fp, dtype=np.int64)
    k = np.ascontiguousarray(k_fp, dtype=np.int64)
    v = np.ascontiguousarray(v_fp, dtype=np.int64)
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError(f"prefill attn shapes: q{q.shape} k{k.shape} v{v.shape}")
    H, M, hd = q.shape
    Hkv, L, hd_k = k.shape
    if hd_k != hd or v.shape != (Hkv, L, hd) or L != int(start) + M:
        raise ValueError(f"prefill attn shape/length mismatch: q{q.shape} k{k.shape} v{v.shape} start={start}")
    out = np.empty((H, M, hd), dtype=np.int64)
    rc = lib.bonsai_attention_prefill_gpu(q.ctypes.data, k.ctypes.data, v.ctypes.data, H, Hkv, hd, M, L, int(start),
                                          int(frac), int(inv_sqrt_fp), out.ctypes.data)
    return None if rc != 0 else out


def attention_decode_batched_gpu(q_fp, Kc, Vc, lengths, frac, inv_sqrt_fp):
    """Batched M=1 decode attention (gpu_native.py:449-468): q (B, H, hd), K/V padded (B, Hkv, cap, hd)."""
    lib = _dev()
    if lib is None:
        return None
    q = np.ascontiguousarray(q_fp, dtype=np.int64)
    K = np.ascontiguousarray(Kc, dtype=np.int64)
    V = np.ascontiguousarray(Vc, dtype=np.int64)
    L = np.ascontiguousarray(np.asarray(lengths, dtype=np.int64))
    B, H, hd = q.shape
    _, Hkv, cap, _ = K.shape
    out = np.empty((B, H, hd), dtype=np.int64)
    rc = lib.bonsai_attention_decode_batched_gpu(q.ctypes.data, K.ctypes.data, V.ctypes.data, L.ctypes.data, B, H,
                                                 Hkv, hd, cap, int(frac), int(inv_sqrt_fp), out.ctypes.data)
    return None if rc != 0 else out


def monolith_available() -> bool:
    return _dev() is not None


def batched_decode_available() -> bool:
    return _dev() is not None


def buf_upload_i64(arr: np.ndarray) -> "int | None":
    """Upload an int64 array once; handle >= 0 or None (gpu_native.py:549-556)."""
    lib = _dev()
    if lib is None:
        return None
    a = np.ascontiguousarray(np.asarray(arr, dtype=np.int64).ravel())
    h = lib.bonsai_buf_upload_i64(a.ctypes.data, a.size)
    return None if int(h) < 0 else int(h)


def _handle_arrays(w, g):
    return {k: np.ascontiguousarray(np.asarray(v, dtype=np.int64)) for k, v in
            dict(wq=w["wq"], wk=w["wk"], wv=w["wv"], wo=w["wo"], w1=w["w1"], wu=w["wu"], w2=w["w2"],
                 n1g=g["n1g"], n2g=g["n2g"], qng=g["qng"], kng=g["kng"]).items()}


_ORDER = ("wq", "wk", "wv", "wo", "w1", "wu", "w2", "n1g", "n2g", "qng", "kng")


def prefill_forward_gpu(x_embed, dims, w, g, frac, eps, inv_sqrt_fp, *, export_kv=False):
    """Whole-prefill monolith (gpu_native.py:559-595): last-row logits, optionally the per-layer KV
    (n_layers, Hkv, T, hd) int64."""
    lib = _dev()
    if lib is None:
        return (None, None, None) if export_kv else None
    T, d, n_layers, H, Hkv, hd, dff = dims
    x = np.ascontiguousarray(np.asarray(x_embed, dtype=np.int64))
    a = _handle_arrays(w, g)
    out = np.empty((int(w["out_head_vocab"]),), dtype=np.int64)
    k_arr = v_arr = None
    if export_kv:
        k_arr = np.empty((n_layers, Hkv, T, hd), dtype=np.int64)
        v_arr = np.empty((n_layers, Hkv, T, hd), dtype=np.int64)
    rc = lib.bonsai_prefill_forward_gpu(
        x.ctypes.data, T, d, n_layers, H, Hkv, hd, dff, int(frac), int(eps), int(inv_sqrt_fp),
        *[a[k].ctypes.data for k in _ORDER], int(g["finalg"]), int(w["out_head"]), int(g["cos_h"]), int(g["sin_h"]),
        out.ctypes.data, None if k_arr is None else k_arr.ctypes.data, None if v_arr is None else v_arr.ctypes.data)
    if rc != 0:
        return (None, None, None) if export_kv else None
    return (out, k_arr, v_arr) if export_kv else out


def decode_ctx_create(dims, w, g, frac, eps, inv_sqrt_fp, cap):
    """Device decode context (gpu_native.py:483-506). dims = (B, n_layers, H, Hkv, hd, d, dff, vocab)."""
    lib = _dev()
    if lib is None:
        return None
    B, n_layers, H, Hkv, hd, d, dff, vocab = dims
    a = _handle_arrays(w, g)
    h = lib.bonsai_decode_ctx_create(B, n_layers, H, Hkv, hd, d, dff, int(cap), int(vocab), int(frac), int(eps),
                                     int(inv_sqrt_fp), *[a[k].ctypes.data for k in _ORDER], int(g["finalg"]),
                                     int(w["out_head"]), int(g["cos_h"]), int(g["sin_h"]))
    return None if int(h) < 0 else int(h)


def decode_ctx_seed_seq(ctx_h, b, k_arr, v_arr):
    """Seed sequence b's prefilled KV, each (n_layers, Hkv, Lb, hd) int64 (gpu_native.py:509-521)."""
    lib = _dev()
    if lib is None:
        return False
    k = np.ascontiguousarray(np.asarray(k_arr, dtype=np.int64))
    v = np.ascontiguousarray(np.asarray(v_arr, dtype=np.int64))
    return lib.bonsai_decode_ctx_seed_seq(int(ctx_h), int(b), k.ctypes.data, v.ctypes.data, int(k.shape[2])) == 0


def decode_step(ctx_h, x_in, pos, vocab):
    """One M=B decode step (gpu_native.py:524-538): logits (B, vocab) or None."""
    lib = _dev()
    if lib is None:
        return None
    x = np.ascontiguousarray(np.asarray(x_in, dtype=np.int64))
    p = np.ascontiguousarray(np.asarray(pos, dtype=np.int64))
    out = np.empty((x.shape[0], int(vocab)), dtype=np.int64)
    rc = lib.bonsai_decode_step(int(ctx_h), x.ctypes.data, p.ctypes.data, out.ctypes.data)
    return None if rc != 0 else out


def decode_ctx_free(ctx_h):
    lib = _dev()
    if lib is not None:
        lib.bonsai_decode_ctx_free(int(ctx_h))
