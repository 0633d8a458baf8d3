"""Device integer samplers behind the reference's sampler interface (gfx950).

Mirrors ``bonsai/src/trinote/infer_int/sampler.py``: ``sample_token(logits_row, cfg, position, frac_bits,
history_ids=None)`` (:403-437) with the same config fields (``SamplerConfig`` :44-63, duck-typed: any object with
``mode, temperature, top_k, top_p, min_p, seed, rep_penalty, no_repeat_ngram`` and the optional committed
``*_fp_committed`` ints), the same committed fixed-point conversions (``inv_temp_fp`` :214-226, ``top_p_fp``
:229-231, ``min_p_fp`` :234-237, ``_resolve_fp`` :247-258) and the same failure behaviour (``ValueError`` for
settings ``validate_sampler_config`` rejects, ``OverflowError`` when temperature scaling would overflow int64).
The distribution, truncation, SHA-256 draw and selection all run on the device (``imie_sample_token``);
``sample_rows_dev`` samples device-resident logits rows without a host copy. There is no CPU fallback: a missing
library raises.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

MODES = {"greedy": 0, "temp": 1, "top_k": 2, "top_p": 3, "min_p": 4}


class SamplerConfigC(ctypes.Structure):
    """``ImieSamplerConfig`` (include/imie_bonsai.h)."""
    _fields_ = [(n, ctypes.c_int64) for n in ("mode", "frac", "inv_temp", "top_k", "top_p", "min_p", "rep_penalty",
                                              "no_repeat_ngram", "seed")]


def inv_temp_fp(temperature: float, frac_bits: int) -> int:
    if temperature <= 0:
        raise ValueError("temperature must be > 0")
    v = round((1 << frac_bits) / float(temperature))
    if v >= (1 << 62):
        raise ValueError("temperature too small for fixed-point sampling — use greedy for argmax")
    return int(v)


def top_p_fp(top_p: float, frac_bits: int) -> int:
    return int(round(float(top_p) * (1 << frac_bits)))


def min_p_fp(min_p: float, frac_bits: int) -> int:
    return int(round(float(min_p) * (1 << frac_bits)))


def _validate(cfg) -> None:
    """validate_sampler_config (sampler.py:71-91)."""
    mode = cfg.mode
    if mode not in MODES:
        raise ValueError(f"unsupported sampler mode {mode!r}")
    if mode != "greedy" and cfg.temperature <= 0:
        raise ValueError("temperature must be > 0 for sampling modes")
    if mode == "top_k" and cfg.top_k <= 0:
        raise ValueError("top_k must be > 0 for top_k sampling")
    if mode == "top_p" and not (0.0 < cfg.top_p <= 1.0):
        raise ValueError("top_p must be in (0, 1] for top_p sampling")
    if mode == "min_p" and not (0.0 < cfg.min_p <= 1.0):
        raise ValueError("min_p must be in (0, 1] for min_p sampling")
    if cfg.top_k < 0 or not (0.0 <= cfg.min_p <= 1.0) or cfg.rep_penalty < 0 or cfg.no_repeat_ngram < 0:
        raise ValueError("invalid sampler settings")


def config_c(cfg, frac_bits: int) -> SamplerConfigC:
    """The committed fixed-point settings of a SamplerConfig (receipt/v2 ints verbatim when present)."""
    _validate(cfg)
    if cfg.mode == "greedy":
        itf, tpf, mpf = 1 << frac_bits, 1 << frac_bits, 0
    else:
        itf = getattr(cfg, "inv_temp_fp_committed", None)
        itf = inv_temp_fp(cfg.temperature, frac_bits) if itf is None else int(itf)
        tpf = getattr(cfg, "top_p_fp_committed", None)
        if cfg.mode in ("top_k", "top_p"):               # _truncate reads it in these modes only (sampler.py:423)
            tpf = top_p_fp(cfg.top_p, frac_bits) if tpf is None else int(tpf)
        else:
            tpf = 1 << frac_bits
        mpf = getattr(cfg, "min_p_fp_committed", None)
        mpf = min_p_fp(cfg.min_p, frac_bits) if mpf is None else int(mpf)
    seed = int(cfg.seed) & ((1 << 64) - 1)              # the draw keys on the low 64 bits (sampler.py:291)
    seed = seed - (1 << 64) if seed >= (1 << 63) else seed
    return SamplerConfigC(MODES[cfg.mode], int(frac_bits), itf, int(cfg.top_k), tpf, mpf, int(cfg.rep_penalty),
                          int(cfg.no_repeat_ngram), seed)


def sample_token(logits_row, cfg, position: int, frac_bits: int, history_ids=None) -> int:
    """One token, byte-identical to the reference sample_token for every mode."""
    lib = _lib.lib()
    row = np.ascontiguousarray(np.asarray(logits_row, dtype=np.int64).reshape(-1))
    c = config_c(cfg, frac_bits)
    hist = None
    if (cfg.rep_penalty or cfg.no_repeat_ngram) and history_ids is not None:
        hist = np.ascontiguousarray(np.asarray(list(history_ids), dtype=np.int64))
    tok = ctypes.c_int64()
    rc = lib.imie_sample_token(row.ctypes.data, row.shape[0], ctypes.byref(c),
                               hist.ctypes.data if hist is not None and hist.size else None,
                               0 if hist is None else int(hist.size), int(position), ctypes.byref(tok))
    if rc == 2:
        raise OverflowError("temperature scaling overflows int64; temperature too small for these logits")
    if rc != 0:
        raise ValueError(f"imie_sample_token failed (rc {rc}): {_lib.last_error()}")
    return int(tok.value)


def sample_rows_dev(logits, cfg, frac_bits: int, positions, history=None, history_len=None, stream=None):
    """Tokens for device logits rows (torch int64 (rows, vocab)); positions / history_len: device int64 (rows,),
    history: device int64 (rows, hist_ld). Returns (tokens, status) device tensors; status != 0 flags the
    temperature guard (2) or a history token outside the vocabulary (1). Asynchronous on `stream`."""
    import torch
    lib = _lib.lib()
    rows, vocab = logits.shape
    c = config_c(cfg, frac_bits)
    tokens = torch.empty(rows, dtype=torch.int64, device=logits.device)
    status = torch.zeros(1, dtype=torch.int32, device=logits.device)
    hp = history.data_ptr() if history is not None else None
    hld = history.shape[1] if history is not None else 0
    lp = history_len.data_ptr() if history_len is not None else None
    st = stream if stream is not None else torch.cuda.current_stream()
    rc = lib.imie_sample_dev(logits.data_ptr(), rows, vocab, logits.stride(0), ctypes.byref(c), hp, hld, lp,
                             positions.data_ptr(), tokens.data_ptr(), status.data_ptr(), ctypes.c_void_p(st.cuda_stream))
    if rc != 0:
        raise ValueError(f"imie_sample_dev failed (rc {rc}): {_lib.last_error()}")
    return tokens, status
