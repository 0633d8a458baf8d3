"""Receipt re-execution: full, sampled-audit, challenged and resampled verification of a committed Bonsai turn
(``bonsai/src/trinote/infer_int/verify.py:27-272``), on the device (``DeviceVerifier``) or on the host CPU,
independent of the GPU producer (``CpuVerifier``).

A receipt commits ``inputIds`` and ``outputIds``; the verifier re-derives every output token from the artifact and
checks it. The strategies, their names, the result dictionaries and the edge rules follow the reference:

* ``verify_greedy``: one teacher-forced prefill of input + output when the turn fits the effective window
  (``min(context_len, RoPE rows)``), else a per-position sliding window over the clamped prefix; with
  ``rep_penalty_fp`` / ``no_repeat_ngram`` the penalty is applied to the row before the lowest-index argmax, with
  the full committed prefix as history. With ``receipt_verify_cached_threshold`` set, long turns replay the
  cached decode instead; ``receipt_verify_strategy`` overrides either way.
* ``verify_sampled``: ``k`` positions chosen by ``numpy.random.Generator(Philox(key=seed)).choice`` (the same
  deterministic audit sample as the reference).
* ``challenge_position``: prefill exactly the committed prefix (engine-clamped) and read its last row.
* ``verify_resample``: each output token must equal the committed sampler's draw at the absolute position
  ``len(input) + i`` with the committed prefix as history.
* Every teacher-forced position carries ``logitsDigest``: SHA-256 of the raw int64 row (little endian).

MI355X design: the artifact is resident (``artifact.register_artifact``), the prefill runs the device layers over
all T positions, the LM head writes the (T, vocab) logits into HBM, and the selection (``imie_sample_dev``: argmax,
penalties, or the seeded sampler) and the row digests (``imie_logits_digest_dev``) run on the device over the rows
that predict output tokens. Only token ids and 32-byte digests cross PCIe (below 64 rows the rows themselves are
hashed on the host, which is faster than one serial device SHA-256 lane). The cached replay runs the device decode
loop (``imie_net_decode_dev`` / ``imie_net_decode_sampled_dev``); the device verifier has no host compute path.
"""
from __future__ import annotations

import ctypes
import hashlib
from types import SimpleNamespace

import numpy as np

from . import _lib
from . import artifact as _artifact


def _greedy_cfg(rep_penalty_fp: int, no_repeat_ngram: int):
    return SimpleNamespace(mode="greedy", temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, seed=0,
                           rep_penalty=int(rep_penalty_fp), no_repeat_ngram=int(no_repeat_ngram))


class DeviceVerifier:
    """A Bonsai artifact resident on one GPU for receipt re-execution (the ``model`` the verify functions take).

    ``cfg`` carries ``frac`` and ``context_len`` like the reference model; ``artifact`` is the loaded artifact."""

    # The reference model switches to cached replay at 64 outputs (reference_bonsai.py:783) because its host
    # all-position head is costly. On the device the teacher-forced prefill is ~9x faster than the replay at the
    # 8B shape (512 + 512 tokens: 0.17 s against 1.56 s), so "auto" stays teacher-forced whenever the turn fits;
    # "cached-replay" can still be selected explicitly.
    receipt_verify_cached_threshold = None
    receipt_verify_strategy = "auto"
    DIGEST_DEVICE_MIN_ROWS = 64

    def __init__(self, artifact: dict, *, page: int = 64):
        import torch
        from .resident import ResidentNet
        self.torch = torch
        self.artifact = artifact
        self.cfg = dict(artifact["config"])
        self.cfg.setdefault("frac", 16)
        self.cfg.setdefault("context_len", int(artifact["cos_fp"].shape[0]))
        self.dims = _artifact.dims(artifact)
        self.eff = min(int(self.cfg["context_len"]), int(artifact["cos_fp"].shape[0]))
        self.vocab = self.dims["vocab"]
        w, g = _artifact.register_artifact(artifact)
        d = self.dims
        self.net = ResidentNet(B=1, n_layers=d["n_layers"], H=d["H"], Hkv=d["Hkv"], hd=d["hd"], d=d["d"],
                               dff=d["dff"], cap=self.eff, w=w, g=g, frac=d["frac"], page=page, kv32=True)
        self.ebits = torch.from_numpy(np.ascontiguousarray(artifact["embed_bits"], dtype=np.uint8)).cuda()
        self.escale = torch.from_numpy(np.ascontiguousarray(artifact["embed_scale_fp"], dtype=np.int64)).cuda()
        self.lib = _lib.lib()

    # ---- device primitives ----------------------------------------------------------------------------------
    def _check(self, what: str) -> None:
        st = self.net.status()
        if st != 0:
            raise RuntimeError(f"{what}: the device producer refused the turn (status {st}); it cannot be "
                               f"re-executed exactly on this producer")

    def _embed(self, ids):
        t = self.torch
        ids_d = t.tensor(np.asarray(ids, dtype=np.int64), device="cuda")
        if int(ids_d.min()) < 0 or int(ids_d.max()) >= self.vocab:
            raise ValueError("token id outside the vocabulary")
        x = t.empty((len(ids), self.dims["d"]), dtype=t.int64, device="cuda")
        rc = self.lib.imie_embed_dev(ctypes.c_void_p(self.ebits.data_ptr()), ctypes.c_void_p(self.escale.data_ptr()),
                                     self.dims["d"] // 128, ctypes.c_void_p(ids_d.data_ptr()), len(ids),
                                     ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(self.net.stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"embedding rc={rc}")
        return x

    def _prefill(self, ids):
        """Fresh cache, all layers over ids at positions 0..T-1; returns the hidden rows (T, d) on the device."""
        T = len(ids)
        if not 0 < T <= self.eff:
            raise ValueError(f"prefill of {T} tokens outside (0, {self.eff}]")
        self.net.reset()
        self.net.stream.wait_stream(self.torch.cuda.current_stream())
        x = self._embed(ids)
        self.net.forward(x, [0], T)
        self._check("prefill")
        return x

    def logits_dev(self, ids, last_only: bool = False):
        """(T, vocab) int64 logits on the device (or the last row only, (1, vocab))."""
        x = self._prefill(ids)
        if last_only:
            x = x[-1:].contiguous()
        logits, _ = self.net.head(x, x.shape[0], argmax=False)
        self._check("head")
        return logits

    def teacher_forced_logits(self, ids) -> np.ndarray:
        return self.logits_dev(list(ids)).cpu().numpy()

    def take_rows(self, full, idx):
        return full.index_select(0, self.torch.tensor(list(idx), dtype=self.torch.int64, device="cuda"))

    def cat_rows(self, rows):
        return self.torch.cat(rows, 0)

    def forward(self, ids) -> np.ndarray:
        return self.teacher_forced_logits(ids)

    def select(self, rows_dev, cfg, positions, histories):
        """Tokens for device rows under a sampler config; histories[i] is row i's committed prefix."""
        from .sampler_gpu import sample_rows_dev
        t = self.torch
        R = rows_dev.shape[0]
        pos = t.tensor(np.asarray(positions, dtype=np.int64), device="cuda")
        hist = hlen = None
        if cfg.rep_penalty or cfg.no_repeat_ngram:
            ld = max(1, max(len(h) for h in histories))
            hh = np.zeros((R, ld), dtype=np.int64)
            for i, h in enumerate(histories):
                hh[i, :len(h)] = h
            hist = t.from_numpy(hh).cuda()
            hlen = t.tensor([len(h) for h in histories], dtype=t.int64, device="cuda")
        tokens, status = sample_rows_dev(rows_dev, cfg, int(self.cfg["frac"]), pos, hist, hlen)
        st = int(status.item())
        if st == 2:
            raise OverflowError("temperature scaling overflows int64; temperature too small for these logits")
        if st != 0:
            raise ValueError(f"device sampler rejected the committed history (status {st})")
        return [int(v) for v in tokens.cpu().numpy()]

    def digests(self, rows_dev) -> list[str]:
        """Row digests: on the device from 64 rows up (one lane per row, ~61 ms for any count up to thousands
        at vocab 151,936); below that the rows are copied and hashed on the host (~1 ms per row)."""
        if rows_dev.shape[0] >= self.DIGEST_DEVICE_MIN_ROWS:
            return logits_digest_dev(rows_dev)
        return [logits_digest(r) for r in rows_dev.cpu().numpy()]

    def replay(self, input_ids, n_out: int, cfg=None):
        """Cached decode replay: prefill input[:-1], then n_out device decode steps from input[-1]; the greedy
        loop, or the sampled loop (cfg) with the committed history and the draw keyed by len(history)."""
        t = self.torch
        n_in = len(input_ids)
        if n_in == 0:
            raise ValueError("cached replay needs a non-empty prompt")
        if n_in + n_out - 1 > self.eff:
            raise ValueError("cached replay exceeds the exact context window")
        self.net.reset()
        self.net.stream.wait_stream(t.cuda.current_stream())
        if n_in > 1:
            x = self._embed(input_ids[:-1])
            self.net.forward(x, [0], n_in - 1)
            self._check("replay prefill")
        ids = t.tensor([int(input_ids[-1])], dtype=t.int64, device="cuda")
        t.cuda.current_stream().synchronize()
        if cfg is None:
            _, hist = self.net.decode(self.ebits, self.escale, ids, n_out, graph=n_out > 1)
            self.net.stream.synchronize()
            self._check("replay")
            return [int(v) for v in hist[:, 0].cpu().numpy()]
        hist = t.zeros((1, n_in + n_out), dtype=t.int64, device="cuda")
        hist[0, :n_in] = t.tensor(np.asarray(input_ids, dtype=np.int64), device="cuda")
        hlen = t.tensor([n_in], dtype=t.int64, device="cuda")
        self.torch.cuda.current_stream().synchronize()
        self.net.decode_sampled(self.ebits, self.escale, ids, n_out, cfg, int(self.cfg["frac"]), hist, hlen,
                                graph=n_out > 1)
        self.net.stream.synchronize()
        self._check("replay")
        return [int(v) for v in hist[0, n_in:].cpu().numpy()]

    def close(self) -> None:
        from . import gpu_native
        self.net.close()
        gpu_native.q1_free_weights()


class CpuVerifier:
    """The same verifier on the host CPU: the ``model`` the verify functions take, re-deriving turns with the
    library's host forward (``imie_cpu_forward``) and host sampler (``imie_cpu_sample_token``), which share no code
    with the device producer. This is the reference's verifier role (verify.py:156-272 on its CPU reference engine):
    a counterparty re-checks a receipt without trusting the GPU that produced it. It has no cached replay (the
    strategies then stay teacher-forced, and an explicit ``cached-replay`` is refused as for any model without an
    exact cached generator). ``threads`` = 0 uses every hardware thread."""

    receipt_verify_cached_threshold = None
    receipt_verify_strategy = "auto"

    def __init__(self, artifact: dict, *, threads: int = 0):
        self.lib = _lib.lib()
        self.artifact = artifact
        self.cfg = dict(artifact["config"])
        self.cfg.setdefault("frac", 16)
        self.cfg.setdefault("context_len", int(artifact["cos_fp"].shape[0]))
        d = _artifact.dims(artifact)
        self.dims = d
        self.eff = min(int(self.cfg["context_len"]), int(artifact["cos_fp"].shape[0]))
        self.vocab = d["vocab"]
        c = lambda a, dt: np.ascontiguousarray(np.asarray(a), dtype=dt)
        keep = []                                          # the host model borrows these arrays

        def ptr(a):
            keep.append(a)
            return a.ctypes.data

        layers = artifact["layers"]
        wb = (ctypes.c_void_p * (7 * len(layers)))(*[ptr(c(l[f"{p}_bits"], np.uint8)) for l in layers
                                                      for p in _artifact.PROJ])
        ws = (ctypes.c_void_p * (7 * len(layers)))(*[ptr(c(l[f"{p}_scale_fp"], np.int64)) for l in layers
                                                      for p in _artifact.PROJ])
        gk = ("n1_gain_fp", "n2_gain_fp", "q_norm_gain_fp", "k_norm_gain_fp")
        gs = (ctypes.c_void_p * (4 * len(layers)))(*[ptr(c(l[k], np.int64)) for l in layers for k in gk])
        cos, sin = c(artifact["cos_fp"], np.int64), c(artifact["sin_fp"], np.int64)
        inv = int(round((1.0 / np.sqrt(d["hd"])) * (1 << d["frac"])))
        h = self.lib.imie_cpu_model_create(d["n_layers"], d["H"], d["Hkv"], d["hd"], d["d"], d["dff"], d["vocab"],
                                           d["frac"], 1, inv, wb, ws, gs, ptr(c(artifact["embed_bits"], np.uint8)),
                                           ptr(c(artifact["embed_scale_fp"], np.int64)),
                                           ptr(c(artifact["output_bits"], np.uint8)),
                                           ptr(c(artifact["output_scale_fp"], np.int64)),
                                           ptr(c(artifact["final_norm_gain_fp"], np.int64)), ptr(cos), ptr(sin),
                                           int(cos.shape[0]))
        if h < 0:
            raise ValueError("imie_cpu_model_create refused the artifact's shapes")
        self.h, self._keep = int(h), (keep, wb, ws, gs)
        self.lib.imie_cpu_set_threads(int(threads))

    def logits_dev(self, ids, last_only: bool = False) -> np.ndarray:
        ids = np.ascontiguousarray(np.asarray(list(ids), dtype=np.int64))
        if not 0 < ids.size <= self.eff:
            raise ValueError(f"prefill of {ids.size} tokens outside (0, {self.eff}]")
        out = np.empty((1 if last_only else ids.size, self.vocab), dtype=np.int64)
        rc = self.lib.imie_cpu_forward(self.h, ids.ctypes.data, ids.size, 1 if last_only else 0, out.ctypes.data)
        if rc == 1:
            raise ValueError("token id outside the vocabulary")
        if rc == 2:
            raise OverflowError("the reference forward raises on this turn (attention / RoPE int64 envelope)")
        if rc != 0:
            raise OverflowError(f"the reference forward raises on this turn (RMSNorm envelope, rc {rc})")
        return out

    def teacher_forced_logits(self, ids) -> np.ndarray:
        return self.logits_dev(ids)

    def forward(self, ids) -> np.ndarray:
        return self.logits_dev(ids)

    def take_rows(self, full, idx):
        return full[np.asarray(list(idx), dtype=np.int64)]

    def cat_rows(self, rows):
        return np.concatenate(rows, 0)

    def select(self, rows, cfg, positions, histories):
        from .sampler_gpu import config_c
        c = config_c(cfg, int(self.cfg["frac"]))
        out = []
        for r, pos, hist in zip(rows, positions, histories):
            row = np.ascontiguousarray(r, dtype=np.int64)
            hh = np.ascontiguousarray(np.asarray(hist, dtype=np.int64))
            use = (cfg.rep_penalty or cfg.no_repeat_ngram) and hh.size
            tok = ctypes.c_int64()
            rc = self.lib.imie_cpu_sample_token(row.ctypes.data, row.shape[0], ctypes.byref(c),
                                                hh.ctypes.data if use else None, int(hh.size) if use else 0,
                                                int(pos), ctypes.byref(tok))
            if rc == 2:
                raise OverflowError("temperature scaling overflows int64; temperature too small for these logits")
            if rc != 0:
                raise ValueError(f"host sampler rejected the committed history (rc {rc})")
            out.append(int(tok.value))
        return out

    def digests(self, rows) -> list[str]:
        return [logits_digest(r) for r in rows]

    def close(self) -> None:
        if self.h >= 0:
            self.lib.imie_cpu_model_free(self.h)
            self.h = -1


def logits_digest(row) -> str:
    """SHA-256 of a host row's little-endian int64 bytes (sampler.py:421-425)."""
    return hashlib.sha256(np.ascontiguousarray(row, dtype="<i8").tobytes()).hexdigest()


def logits_digest_dev(rows_dev) -> list[str]:
    """SHA-256 of each device row (torch int64 (R, vocab), unit inner stride) computed on the device."""
    import torch
    R, V = rows_dev.shape
    if rows_dev.stride(1) != 1:
        raise ValueError("rows must be contiguous along the vocabulary")
    out = torch.empty((R, 32), dtype=torch.uint8, device=rows_dev.device)
    rc = _lib.lib().imie_logits_digest_dev(ctypes.c_void_p(rows_dev.data_ptr()), R, V, rows_dev.stride(0),
                                           ctypes.c_void_p(out.data_ptr()),
                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    if rc != 0:
        raise RuntimeError(f"imie_logits_digest_dev rc={rc}")
    return [bytes(r).hex() for r in out.cpu().numpy()]


# ---- strategy selection (verify.py:60-103) -------------------------------------------------------------------------
def _cached_threshold(model):
    th = getattr(model, "receipt_verify_cached_threshold", None)
    if th is None or not hasattr(model, "replay"):
        return None
    return max(1, int(th))


def _has_replay(model) -> bool:
    return hasattr(model, "replay")


def _strategy(model, n_out: int) -> str:
    sel = str(getattr(model, "receipt_verify_strategy", "auto") or "auto")
    if sel not in {"auto", "teacher-forced", "cached-replay"}:
        raise ValueError(f"unknown receipt verification strategy {sel!r}")
    if sel == "teacher-forced":
        return sel
    th = _cached_threshold(model)
    if sel == "cached-replay":
        if not _has_replay(model):
            raise ValueError("cached-replay requested but this model has no exact cached generator")
        return sel
    return "cached-replay" if th is not None and n_out >= th else "teacher-forced"


def _replay_positions(input_ids, output_ids, replayed):
    n_in = len(input_ids)
    ok = len(replayed) == len(output_ids)
    positions = []
    for i, expected in enumerate(output_ids):
        pred = int(replayed[i]) if i < len(replayed) else None
        match = pred == int(expected)
        ok = ok and match
        positions.append({"position": n_in + i, "expected": int(expected), "predicted": pred, "match": match})
    return ok, positions


def _check_cached(model, seq, strategy):
    if strategy == "cached-replay" and len(seq) > model.eff and \
            getattr(model, "receipt_verify_strategy", "auto") == "cached-replay":
        raise ValueError("cached-replay was explicitly selected, but the committed turn exceeds the exact context "
                         "window")
    return strategy == "cached-replay" and len(seq) <= model.eff


def _rows(model, input_ids, output_ids, idx):
    """Device rows predicting output[i] for i in idx: one prefill when the turn fits, else one clamped prefill
    per position (verify.py:114-136). Returns (rows (len(idx), vocab) device, strategy suffix)."""
    n_in = len(input_ids)
    if any(n_in + i - 1 < 0 for i in idx):
        raise ValueError("no predicting row for output[0] with empty inputIds — a generation receipt must commit a "
                         "non-empty prompt")
    seq = list(input_ids) + list(output_ids)
    if len(seq) <= model.eff:
        full = model.logits_dev(seq)
        return model.take_rows(full, [n_in + i - 1 for i in idx]), "full"
    rows = [model.logits_dev(seq[:n_in + i][-model.eff:], last_only=True) for i in idx]
    return model.cat_rows(rows), "sliding"


def _teacher_forced(model, input_ids, output_ids, idx, cfg, keyed: bool):
    rows, kind = _rows(model, input_ids, output_ids, idx)
    n_in = len(input_ids)
    seq = list(input_ids) + list(output_ids)
    hists = [seq[:n_in + i] for i in idx]
    pred = model.select(rows, cfg, [n_in + i for i in idx] if keyed else [0] * len(idx), hists)
    digs = model.digests(rows)
    ok, positions = True, []
    for j, i in enumerate(idx):
        match = pred[j] == int(output_ids[i])
        ok = ok and match
        positions.append({"position": n_in + i, "expected": int(output_ids[i]), "predicted": pred[j],
                          "match": match, "logitsDigest": digs[j]})
    return ok, positions, kind


# ---- public verification API (verify.py:156-272) -------------------------------------------------------------------
def verify_greedy(model, input_ids, output_ids, *, rep_penalty_fp: int = 0, no_repeat_ngram: int = 0) -> dict:
    input_ids, output_ids = [int(v) for v in input_ids], [int(v) for v in output_ids]
    if not output_ids:
        return {"ok": True, "checked": 0, "positions": [], "strategy": "greedy-full"}
    seq = input_ids + output_ids
    if _check_cached(model, seq, _strategy(model, len(output_ids))):
        cfg = _greedy_cfg(rep_penalty_fp, no_repeat_ngram) if (rep_penalty_fp or no_repeat_ngram) else None
        ok, positions = _replay_positions(input_ids, output_ids, model.replay(input_ids, len(output_ids), cfg))
        return {"ok": ok, "checked": len(output_ids), "positions": positions, "strategy": "greedy-cached-replay",
                "logitsDigest": None, "fracBits": int(model.cfg["frac"])}
    ok, positions, kind = _teacher_forced(model, input_ids, output_ids, list(range(len(output_ids))),
                                          _greedy_cfg(rep_penalty_fp, no_repeat_ngram), keyed=False)
    return {"ok": ok, "checked": len(positions), "positions": positions, "strategy": f"greedy-{kind}"}


def verify_sampled(model, input_ids, output_ids, *, k: int, seed: int = 0, rep_penalty_fp: int = 0,
                   no_repeat_ngram: int = 0) -> dict:
    input_ids, output_ids = [int(v) for v in input_ids], [int(v) for v in output_ids]
    n = len(output_ids)
    if n == 0:
        return {"ok": True, "checked": 0, "positions": [], "strategy": "greedy-sampled"}
    k = max(1, min(k, n))
    rng = np.random.Generator(np.random.Philox(key=seed))
    chosen = sorted(int(j) for j in rng.choice(n, size=k, replace=False))
    ok, positions, _ = _teacher_forced(model, input_ids, output_ids, chosen,
                                       _greedy_cfg(rep_penalty_fp, no_repeat_ngram), keyed=False)
    return {"ok": ok, "checked": k, "of": n, "positions": positions, "strategy": "greedy-sampled"}


def challenge_position(model, input_ids, output_ids, i: int, *, rep_penalty_fp: int = 0,
                       no_repeat_ngram: int = 0) -> dict:
    input_ids, output_ids = [int(v) for v in input_ids], [int(v) for v in output_ids]
    if not 0 <= i < len(output_ids):
        raise IndexError(i)
    full_prefix = input_ids + output_ids[:i]
    row = model.logits_dev(full_prefix[-model.eff:], last_only=True)
    pred = model.select(row, _greedy_cfg(rep_penalty_fp, no_repeat_ngram), [0], [full_prefix])[0]
    return {"position": len(input_ids) + i, "expected": int(output_ids[i]), "predicted": pred,
            "match": pred == int(output_ids[i]), "logitsDigest": model.digests(row)[0],
            "strategy": "greedy-challenge"}


def verify_resample(model, input_ids, output_ids, *, sampler_cfg) -> dict:
    input_ids, output_ids = [int(v) for v in input_ids], [int(v) for v in output_ids]
    if not output_ids:
        return {"ok": True, "checked": 0, "positions": [], "strategy": "resample-full"}
    seq = input_ids + output_ids
    if _check_cached(model, seq, _strategy(model, len(output_ids))):
        ok, positions = _replay_positions(input_ids, output_ids,
                                          model.replay(input_ids, len(output_ids), sampler_cfg))
        return {"ok": ok, "checked": len(output_ids), "positions": positions,
                "strategy": "resample-cached-replay", "logitsDigest": None}
    ok, positions, kind = _teacher_forced(model, input_ids, output_ids, list(range(len(output_ids))), sampler_cfg,
                                          keyed=True)
    return {"ok": ok, "checked": len(positions), "positions": positions, "strategy": f"resample-{kind}"}
