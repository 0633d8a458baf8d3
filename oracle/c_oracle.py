"""ctypes wrapper of ``oracle/liboracle_c.so`` — the C/OpenMP restatement used for large configs (test
infrastructure only). Each function returns exactly what the numpy oracle returns (or raises where it raises);
``tests/test_oracle_c.py`` asserts that equality on random and adversarial inputs."""
from __future__ import annotations

import ctypes
import subprocess
from ctypes import c_int, c_int64, c_void_p
from functools import lru_cache
from pathlib import Path

import numpy as np

from . import fixedpoint as fx

HERE = Path(__file__).resolve().parent
SO = HERE / "liboracle_c.so"


@lru_cache(maxsize=1)
def lib():
    if not SO.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), str(SO)], check=True)
    so = ctypes.CDLL(str(SO))
    so.imo_q1_linear.argtypes = [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p]
    so.imo_rmsnorm.argtypes = [c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p]
    so.imo_attention.argtypes = [c_void_p] * 3 + [c_int64] * 8 + [c_void_p]
    so.imo_qk_linear.argtypes = [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_int, c_void_p]
    so.imo_attention_ld.argtypes = [c_void_p] * 3 + [c_int64] * 9 + [c_void_p]
    so.imo_uniform_fill.argtypes = [ctypes.c_uint64, ctypes.c_uint64, c_int64, c_int64, c_int64, c_int64, c_int64,
                                    ctypes.c_uint64, c_void_p]
    so.imo_silu_mul.argtypes = [c_void_p, c_void_p, c_int64, c_int64, c_void_p]
    so.imo_fp16_fixed.argtypes = [ctypes.c_uint16, c_int]
    so.imo_fp16_fixed.restype = c_int64
    for f in (so.imo_q1_linear, so.imo_rmsnorm, so.imo_attention, so.imo_qk_linear, so.imo_silu_mul,
              so.imo_attention_ld, so.imo_uniform_fill):
        f.restype = c_int
    return so


def _c(a, dt=np.int64):
    return np.ascontiguousarray(a, dtype=dt)


def q1_linear(x, bits, scale, frac):
    x = _c(np.atleast_2d(x))
    b = _c(bits, np.uint8)
    s = _c(scale)
    N, nb = s.shape
    out = np.empty((x.shape[0], N), dtype=np.int64)
    assert lib().imo_q1_linear(x.ctypes.data, b.ctypes.data, s.ctypes.data, x.shape[0], N, nb, int(frac),
                               out.ctypes.data) == 0
    return out


def rmsnorm(x, frac, eps=1, gain=None):
    x = _c(np.atleast_2d(x))
    out = np.empty_like(x)
    g = None if gain is None else _c(gain)
    rc = lib().imo_rmsnorm(x.ctypes.data, x.shape[0], x.shape[1], int(frac), int(eps),
                           None if g is None else g.ctypes.data, out.ctypes.data)
    if rc == 4:
        return fx.rmsnorm(x, frac, eps, gain)        # beyond 128 bits: big-int oracle
    if rc == 2:
        raise OverflowError("rmsnorm gain multiply would overflow int64")
    assert rc == 0
    return out


def silu_mul(gate, up, frac):
    """(silu(gate) * up) >> frac, elementwise, wrapping (fx.mulshift_wrap(fx.silu_wrap(gate), up))."""
    g = _c(gate)
    u = _c(up)
    assert g.shape == u.shape
    out = np.empty(g.shape, dtype=np.int64)
    assert lib().imo_silu_mul(g.ctypes.data, u.ctypes.data, g.size, int(frac), out.ctypes.data) == 0
    return out


def attention_cached(qh, k, v, start, frac, inv_sqrt):
    q = _c(qh)
    k = _c(k)
    v = _c(v)
    H, M, hd = q.shape
    Hkv, L, _ = k.shape
    out = np.empty((H, M, hd), dtype=np.int64)
    rc = lib().imo_attention(q.ctypes.data, k.ctypes.data, v.ctypes.data, H, Hkv, hd, M, L, int(start), int(frac),
                             int(inv_sqrt), out.ctypes.data)
    if rc == 2:
        raise OverflowError("fixed_point_matmul bound exceeded")
    assert rc == 0
    return out


def attention_ld(qh, kbuf, vbuf, L, start, frac, inv_sqrt):
    """attention_cached over the first L rows of per-kv-head row buffers kbuf/vbuf (Hkv, cap, hd), cap >= L."""
    q = _c(qh)
    assert kbuf.flags.c_contiguous and vbuf.flags.c_contiguous and kbuf.dtype == np.int64 == vbuf.dtype
    H, M, hd = q.shape
    Hkv, cap, _ = kbuf.shape
    out = np.empty((H, M, hd), dtype=np.int64)
    rc = lib().imo_attention_ld(q.ctypes.data, kbuf.ctypes.data, vbuf.ctypes.data, H, Hkv, hd, M, int(L), cap,
                                int(start), int(frac), int(inv_sqrt), out.ctypes.data)
    if rc == 2:
        raise OverflowError("fixed_point_matmul bound exceeded")
    assert rc == 0
    return out


def uniform_fill(seed: int, tid: int, out: np.ndarray, rows: int, cols: int, lo: int, hi: int, first: int = 0) -> None:
    """Elements first .. first + rows*cols of the stream of prng.uniform_int(seed, tid, ..., lo, hi), as a (rows,
    cols) block written into the first ``cols`` entries of the first ``rows`` rows of the 2-D int64 array ``out``
    (row stride out.shape[1])."""
    assert out.flags.c_contiguous and out.dtype == np.int64 and out.ndim == 2 and out.shape[1] >= cols
    assert out.shape[0] >= rows
    assert lib().imo_uniform_fill(seed, tid, int(first), rows, cols, out.shape[1], lo, hi - lo, out.ctypes.data) == 0


def qk_linear(raw: np.ndarray, x, out_f: int, nb: int, fw: int, qtype: int):
    w = _c(np.frombuffer(raw, dtype=np.uint8) if isinstance(raw, (bytes, bytearray)) else raw, np.uint8)
    x = _c(np.atleast_2d(x))
    out = np.empty((x.shape[0], out_f), dtype=np.int64)
    rc = lib().imo_qk_linear(w.ctypes.data, x.ctypes.data, x.shape[0], out_f, nb, int(fw), int(qtype),
                             out.ctypes.data)
    if rc == 2:
        raise OverflowError("nmc linear result leaves int64")
    assert rc == 0
    return out


def fp16_fixed(h: int, fw: int) -> int:
    return int(lib().imo_fp16_fixed(int(h), int(fw)))
