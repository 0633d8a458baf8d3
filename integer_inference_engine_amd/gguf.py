"""GGUF readers feeding the resident weight managers (host side, zero-copy).

Behaviour follows the reference importers:

* Bonsai Q1_0 (``bonsai/src/trinote/infer_int/import_bonsai_gguf.py:17-93``): GGML type 41, 18-byte blocks of an
  fp16 scale and 128 sign bits; a 2-D tensor ``[ne0 = in, ne1 = out]`` becomes ``bits (out, in/128, 16)`` and
  ``scale = rint(fp16 * 2^frac)`` as int64, refusing non-finite scales and magnitudes beyond int64 (:69-84).
* F16 / F32 gains to fixed point with the same refusal (:96-97).
* north-mini-code Q4_K / Q6_K (``north-mini-code/src/nmc/gguf.py:77-122``): raw rows, and one expert's contiguous
  slice of a 3-D expert tensor ``[ne0 = in, ne1 = out, n_experts]`` read lazily (only that expert's bytes).

The file format is GGUF v2/v3 (little endian): magic, version, tensor and KV counts, typed KV pairs, tensor infos
(name, dims, type, offset), then the data section at ``general.alignment`` (default 32). Tensor bytes are views of
a read-only memory map; nothing is copied until a caller asks for arrays.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

F32, F16, Q4_K, Q6_K, Q1_0 = 0, 1, 12, 14, 41
QK1_0, Q1_BLOCK = 128, 18
_QK_BLOCK = {Q4_K: (256, 144), Q6_K: (256, 210)}
_SCALAR = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}
_STRING, _ARRAY = 8, 9


class GGUF:
    """Parsed header + memory-mapped data of one GGUF file."""

    def __init__(self, path):
        self.path = Path(path)
        self.buf = np.memmap(self.path, dtype=np.uint8, mode="r")
        self._pos = 0
        if bytes(self.buf[:4]) != b"GGUF":
            raise ValueError(f"{self.path}: not a GGUF file")
        self._pos = 4
        self.version = self._u("I")
        if self.version not in (2, 3):
            raise ValueError(f"{self.path}: unsupported GGUF version {self.version}")
        n_tensors, n_kv = self._u("Q"), self._u("Q")
        self.kv = {}
        for _ in range(n_kv):
            key = self._str()
            self.kv[key] = self._value(self._u("I"))
        self.tensors = {}
        for _ in range(n_tensors):
            name = self._str()
            shape = [self._u("Q") for _ in range(self._u("I"))]
            self.tensors[name] = {"shape": shape, "type": self._u("I"), "offset": self._u("Q")}
        align = int(self.kv.get("general.alignment", 32))
        if align <= 0 or align & (align - 1):
            raise ValueError(f"{self.path}: general.alignment {align} is not a power of two")
        self.data_start = (self._pos + align - 1) // align * align
        for name, t in self.tensors.items():
            t["nbytes"] = _nbytes(name, t["shape"], t["type"])
            end = self.data_start + t["offset"] + t["nbytes"]
            if t["offset"] % align or end > self.buf.size:
                raise ValueError(f"{name}: tensor data out of the file or misaligned")

    # ---- header primitives ----------------------------------------------------------------------------
    def _u(self, fmt):
        n = struct.calcsize("<" + fmt)
        v = struct.unpack_from("<" + fmt, self.buf, self._pos)[0]
        self._pos += n
        return v

    def _str(self):
        n = self._u("Q")
        s = bytes(self.buf[self._pos:self._pos + n]).decode("utf-8")
        self._pos += n
        return s

    def _value(self, t):
        if t == _STRING:
            return self._str()
        if t == _ARRAY:
            et, n = self._u("I"), self._u("Q")
            return [self._value(et) for _ in range(n)]
        if t not in _SCALAR:
            raise ValueError(f"unknown GGUF value type {t}")
        return self._u(_SCALAR[t])

    # ---- tensor access --------------------------------------------------------------------------------
    def raw(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        o = self.data_start + t["offset"]
        return self.buf[o:o + t["nbytes"]]

    def q1_packed(self, name: str, frac: int = 16):
        """Q1_0 2-D tensor -> (bits (out, in/128, 16) uint8, scale (out, in/128) int64 = rint(fp16 * 2^frac))."""
        t = self.tensors[name]
        if t["type"] != Q1_0 or len(t["shape"]) != 2:
            raise ValueError(f"{name}: expected a 2-D Q1_0 tensor, got type {t['type']} shape {t['shape']}")
        in_f, out_f = t["shape"]
        blocks = self.raw(name).reshape(out_f, in_f // QK1_0, Q1_BLOCK)
        scale16 = np.ascontiguousarray(blocks[:, :, :2]).view("<f2").reshape(out_f, in_f // QK1_0)
        return np.ascontiguousarray(blocks[:, :, 2:]), to_fixed(scale16, frac, f"{name} Q1_0 scale")

    def fixed(self, name: str, frac: int = 16) -> np.ndarray:
        """F16 / F32 tensor (flattened) -> int64 rint(x * 2^frac)."""
        t = self.tensors[name]
        if t["type"] not in (F16, F32):
            raise ValueError(f"{name}: expected an F16 / F32 tensor, got type {t['type']}")
        vals = self.raw(name).view("<f2" if t["type"] == F16 else "<f4")
        return to_fixed(vals, frac, f"{name}")

    def quant_rows(self, name: str):
        """Raw Q4_K / Q6_K bytes of a 2-D tensor [in, out] as (bytes (out * nb * block), out, nb, qtype)."""
        t = self.tensors[name]
        if t["type"] not in _QK_BLOCK or len(t["shape"]) != 2:
            raise ValueError(f"{name}: expected a 2-D Q4_K / Q6_K tensor")
        qk, _ = _QK_BLOCK[t["type"]]
        in_f, out_f = t["shape"]
        return self.raw(name), out_f, in_f // qk, (0 if t["type"] == Q4_K else 1)

    def expert_raw(self, name: str, e: int):
        """Expert e of a 3-D Q4_K / Q6_K tensor [in, out, n_experts]: (bytes, out, nb, qtype), only its slice."""
        t = self.tensors[name]
        if t["type"] not in _QK_BLOCK or len(t["shape"]) != 3:
            raise ValueError(f"{name}: expected a 3-D Q4_K / Q6_K expert tensor")
        in_f, out_f, n_e = t["shape"]
        if not 0 <= e < n_e:
            raise IndexError(f"{name}: expert {e} outside [0, {n_e})")
        qk, blk = _QK_BLOCK[t["type"]]
        per = out_f * (in_f // qk) * blk
        o = self.data_start + t["offset"] + e * per
        return self.buf[o:o + per], out_f, in_f // qk, (0 if t["type"] == Q4_K else 1)


def _nbytes(name, shape, tt) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    if tt == F32:
        return 4 * n
    if tt == F16:
        return 2 * n
    if tt == Q1_0:
        if int(shape[0]) % QK1_0:
            raise ValueError(f"{name}: Q1_0 ne0 {shape[0]} not divisible by {QK1_0}")
        return n // QK1_0 * Q1_BLOCK
    if tt in _QK_BLOCK:
        qk, blk = _QK_BLOCK[tt]
        if int(shape[0]) % qk:
            raise ValueError(f"{name}: ne0 {shape[0]} not divisible by {qk}")
        return n // qk * blk
    raise ValueError(f"{name}: unsupported GGML type {tt}")


def to_fixed(x, frac: int, where: str) -> np.ndarray:
    """rint(x * 2^frac) as int64 (round half to even), refusing non-finite values and magnitudes >= 2^63."""
    v = np.asarray(x, dtype=np.float64)
    if not np.all(np.isfinite(v)):
        raise ValueError(f"{where}: non-finite value(s) in the GGUF float data")
    s = v * float(1 << frac)
    if np.any(np.abs(s) >= float(1 << 63)):
        raise ValueError(f"{where}: fixed-point magnitude exceeds int64 at frac={frac}")
    return np.rint(s).astype(np.int64)


def register_q1(gguf: GGUF, names, frac: int = 16) -> dict:
    """Register Q1_0 tensors as resident Bonsai weights (gpu_native.q1_register_weight); {name: handle}."""
    from . import gpu_native
    out = {}
    for n in names:
        bits, scale = gguf.q1_packed(n, frac)
        h = gpu_native.q1_register_weight(bits, scale)
        if h is None:
            raise RuntimeError(f"{n}: resident Q1_0 registration failed")
        out[n] = h
    return out


def register_expert(gguf: GGUF, name: str, e: int) -> int:
    """Register one expert slice of a 3-D Q4_K / Q6_K tensor (qk_gpu.register_weight); the handle."""
    from . import qk_gpu
    raw, out_f, nb, qt = gguf.expert_raw(name, e)
    return qk_gpu.register_weight(np.ascontiguousarray(raw), out_f, nb, qt)
