"""Device-resident Bonsai forward (layers + optional head) over a paged integer KV cache.

Host-side wrapper of the ``imie_net_*`` C-ABI (no reference counterpart; the reference's decode context,
``gpu_native.decode_ctx_*``, is the host-pointer special case). Activations stay in HBM between calls; torch is
used only to own device memory and streams.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

_ORDER = ("wq", "wk", "wv", "wo", "w1", "wu", "w2", "n1g", "n2g", "qng", "kng")


class ResidentNet:
    """B sequences, ``cap`` positions each, ``page`` tokens per KV page, int32 (guarded) or int64 KV."""

    def __init__(self, *, B: int, n_layers: int, H: int, Hkv: int, hd: int, d: int, dff: int, cap: int, w: dict,
                 g: dict, frac: int = 16, eps: int = 1, inv_sqrt: int | None = None, page: int = 64,
                 kv32: bool = True):
        import torch  # device memory owner
        self.torch = torch
        self.lib = _lib.lib()
        if inv_sqrt is None:
            inv_sqrt = int(round((1.0 / np.sqrt(hd)) * (1 << frac)))
        arrs = {k: np.ascontiguousarray(np.asarray(v, dtype=np.int64)) for k, v in
                dict(wq=w["wq"], wk=w["wk"], wv=w["wv"], wo=w["wo"], w1=w["w1"], wu=w["wu"], w2=w["w2"],
                     n1g=g["n1g"], n2g=g["n2g"], qng=g["qng"], kng=g["kng"]).items()}
        h = self.lib.imie_net_create(B, n_layers, H, Hkv, hd, d, dff, cap, frac, eps, inv_sqrt,
                                     *[arrs[k].ctypes.data for k in _ORDER], int(g.get("finalg", -1)),
                                     int(w.get("out_head", -1)), int(g["cos_h"]), int(g["sin_h"]), page,
                                     1 if kv32 else 0)
        if h < 0:
            raise RuntimeError(f"imie_net_create failed: {_lib.last_error()}")
        self.h = int(h)
        self.B, self.d, self.nl, self.Hkv, self.hd = B, d, n_layers, Hkv, hd
        self.vocab = int(w.get("out_head_vocab", 0))
        self.stream = torch.cuda.Stream()

    def _sp(self):
        return ctypes.c_void_p(self.stream.cuda_stream)

    def set_caps(self, caps) -> None:
        """Ragged cache: room for caps[b] positions in sequence b; replaces the cache (lengths restart at 0)."""
        c = np.ascontiguousarray(np.asarray(caps, dtype=np.int64))
        if c.shape != (self.B,):
            raise ValueError(f"caps must have {self.B} entries")
        rc = self.lib.imie_net_set_caps(self.h, c.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"set_caps rc={rc}: {_lib.last_error()}")

    def reset(self) -> None:
        """Every sequence back to length 0; the pools stay allocated."""
        rc = self.lib.imie_net_reset(self.h)
        if rc != 0:
            raise RuntimeError(f"reset rc={rc}: {_lib.last_error()}")

    def fill_kv(self, seed: int, lens, lo: int = -(1 << 20), hi: int = 1 << 20, seq_ids=None) -> None:
        """Seeded synthetic K/V (device-generated) for lens[b] positions of every layer; sets the lengths.
        seq_ids[b] keys sequence b's draw (default b)."""
        ln = np.ascontiguousarray(np.asarray(lens, dtype=np.int64))
        sid = None if seq_ids is None else np.ascontiguousarray(np.asarray(seq_ids, dtype=np.int64))
        rc = self.lib.imie_net_fill_kv(self.h, int(seed), ln.ctypes.data, None if sid is None else sid.ctypes.data,
                                       int(lo), int(hi))
        if rc != 0:
            raise RuntimeError(f"fill_kv rc={rc}: {_lib.last_error()}")

    def seed(self, b: int, k: np.ndarray, v: np.ndarray) -> None:
        """k/v (n_layers, Hkv, Lb, hd) int64."""
        k = np.ascontiguousarray(k, dtype=np.int64)
        v = np.ascontiguousarray(v, dtype=np.int64)
        rc = self.lib.bonsai_decode_ctx_seed_seq(self.h, b, k.ctypes.data, v.ctypes.data, k.shape[2])
        if rc != 0:
            raise RuntimeError(f"seed rc={rc}")

    def forward(self, x, starts, M: int):
        """x: torch int64 (B*M, d) on the device, updated in place. Returns the status word (0 = exact)."""
        st = np.ascontiguousarray(np.asarray(starts, dtype=np.int64))
        self.lib.imie_net_status(self.h, 1, self._sp())
        rc = self.lib.imie_net_forward_dev(self.h, ctypes.c_void_p(x.data_ptr()), st.ctypes.data, int(M), self._sp())
        if rc != 0:
            raise RuntimeError(f"forward rc={rc}: {_lib.last_error()}")
        return self.lib.imie_net_status(self.h, 0, self._sp())

    def head(self, x, rows: int, *, argmax: bool = True):
        t = self.torch
        logits = t.empty((rows, self.vocab), dtype=t.int64, device="cuda")
        ids = t.empty((rows,), dtype=t.int64, device="cuda") if argmax else None
        rc = self.lib.imie_net_head_dev(self.h, ctypes.c_void_p(x.data_ptr()), rows,
                                        ctypes.c_void_p(logits.data_ptr()),
                                        ctypes.c_void_p(ids.data_ptr()) if ids is not None else None, self._sp())
        if rc != 0:
            raise RuntimeError(f"head rc={rc}")
        self.stream.synchronize()
        return logits, ids

    def decode(self, embed_bits, embed_scale, ids, steps: int, *, graph: bool = True, hist=None, logits=None):
        """Greedy decode ``steps`` tokens on the device. embed_bits (vocab, nb, 16) uint8 and embed_scale
        (vocab, nb) int64 torch tensors on the device; ids (B,) int64 device tensor, overwritten with the last
        token. Returns (logits of the last step (B, vocab), hist (steps, B)) as device tensors."""
        t = self.torch
        if logits is None:
            logits = t.empty((self.B, self.vocab), dtype=t.int64, device="cuda")
        if hist is None:
            hist = t.empty((steps, self.B), dtype=t.int64, device="cuda")
        rc = self.lib.imie_net_decode_dev(self.h, ctypes.c_void_p(embed_bits.data_ptr()),
                                          ctypes.c_void_p(embed_scale.data_ptr()), ctypes.c_void_p(ids.data_ptr()),
                                          ctypes.c_void_p(logits.data_ptr()), ctypes.c_void_p(hist.data_ptr()),
                                          int(steps), 1 if graph else 0, self._sp())
        if rc != 0:
            raise RuntimeError(f"decode rc={rc}: {_lib.last_error()}")
        return logits, hist

    def decode_sampled(self, embed_bits, embed_scale, ids, steps: int, cfg, frac: int, hist, hist_len, *,
                       graph: bool = True, logits=None):
        """Sampled decode of ``steps`` tokens on the device (imie_net_decode_sampled_dev). cfg: a SamplerConfig
        (duck-typed, see sampler_gpu); hist (B, hist_ld) int64 device tensor of every sequence's tokens so far,
        hist_len (B,) their counts (both advanced in place); ids (B,) the step's input tokens, overwritten with
        the last drawn token. Returns the last step's logits (B, vocab)."""
        from .sampler_gpu import config_c
        t = self.torch
        if logits is None:
            logits = t.empty((self.B, self.vocab), dtype=t.int64, device="cuda")
        c = config_c(cfg, frac)
        rc = self.lib.imie_net_decode_sampled_dev(self.h, ctypes.c_void_p(embed_bits.data_ptr()),
                                                  ctypes.c_void_p(embed_scale.data_ptr()),
                                                  ctypes.c_void_p(ids.data_ptr()), ctypes.c_void_p(logits.data_ptr()),
                                                  ctypes.byref(c), ctypes.c_void_p(hist.data_ptr()), hist.shape[1],
                                                  ctypes.c_void_p(hist_len.data_ptr()), int(steps), 1 if graph else 0,
                                                  self._sp())
        if rc != 0:
            raise RuntimeError(f"sampled decode rc={rc}: {_lib.last_error()}")
        return logits

    def status(self) -> int:
        return int(self.lib.imie_net_status(self.h, 0, self._sp()))

    def clear_status(self) -> None:
        self.lib.imie_net_status(self.h, 1, self._sp())

    def export_kv(self, layer: int, b: int, count: int):
        k = np.empty((self.Hkv, count, self.hd), dtype=np.int64)
        v = np.empty_like(k)
        self.stream.synchronize()
        rc = self.lib.imie_net_export_kv(self.h, layer, b, count, k.ctypes.data, v.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"export rc={rc}")
        return k, v

    def close(self) -> None:
        if self.h >= 0:
            self.stream.synchronize()
            self.lib.bonsai_decode_ctx_free(self.h)
            self.h = -1
