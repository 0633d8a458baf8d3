"""Bonsai (dense Qwen3, Q1_0) model artifacts: GGUF import, safetensors persistence, digest, device registration.

The on-disk layout is the reference's ``trinote-artifact-bonsai-qwen3/1`` safetensors file
(``bonsai/src/trinote/infer_int/artifact_io_bonsai.py:28-41, 115-160, 192-283``):

* top-level arrays ``embed_bits/embed_scale_fp``, ``output_bits/output_scale_fp``, ``final_norm_gain_fp``,
  ``cos_fp``, ``sin_fp``; per layer ``layers.{i}.<key>`` for the four gains and the seven Q1_0 projections
  (``*_bits`` uint8 (out, in/128, 16), ``*_scale_fp`` int64 (out, in/128));
* one metadata entry ``"trinote"`` = ``json.dumps({"format", "n_layers", "config"[, "provenance"]},
  sort_keys=True)``;
* the digest is SHA-256 of the serialized bytes (the safetensors library's canonical serialization, the same one
  the reference calls), so an artifact written here carries the digest the reference computes for it.

``import_gguf`` follows ``import_bonsai_gguf.py:103-214`` (required keys, integral rope base, context bound,
plain or YaRN RoPE tables, vocab agreement) on top of :mod:`.gguf`. ``register_artifact`` uploads an artifact into
the resident Q1_0 registry and the device buffer table and returns the handle bundles ``ResidentNet`` and the
reference-shaped ``gpu_native`` entry points take (``gpu_native.py:483-595``).

The hybrid Qwen3.5 (27B) artifact format is a different architecture and is refused.
"""
from __future__ import annotations

import hashlib
import json
import os
import tempfile
from pathlib import Path

import numpy as np

from . import gguf as _gguf
from .rope_tables import plain_tables, yarn_tables

FORMAT = "trinote-artifact-bonsai-qwen3/1"
FORMAT_QWEN35 = "trinote-artifact-bonsai-qwen35/1"
TOP_KEYS = ("embed_bits", "embed_scale_fp", "output_bits", "output_scale_fp", "final_norm_gain_fp", "cos_fp",
            "sin_fp")
LAYER_KEYS = ("n1_gain_fp", "n2_gain_fp", "q_norm_gain_fp", "k_norm_gain_fp",
              "wq_bits", "wq_scale_fp", "wk_bits", "wk_scale_fp", "wv_bits", "wv_scale_fp",
              "wo_bits", "wo_scale_fp", "w1_bits", "w1_scale_fp", "wu_bits", "wu_scale_fp",
              "w2_bits", "w2_scale_fp")
PROJ = ("wq", "wk", "wv", "wo", "w1", "wu", "w2")
GAINS = {"n1g": "n1_gain_fp", "n2g": "n2_gain_fp", "qng": "q_norm_gain_fp", "kng": "k_norm_gain_fp"}
MAX_CTX = 1 << 20
_GGUF_PROJ = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "w1": "ffn_gate",
              "wu": "ffn_up", "w2": "ffn_down"}
_GGUF_GAIN = {"n1_gain_fp": "attn_norm", "n2_gain_fp": "ffn_norm", "q_norm_gain_fp": "attn_q_norm",
              "k_norm_gain_fp": "attn_k_norm"}


class ArtifactError(RuntimeError):
    """An artifact that is missing, unreadable or not a dense Bonsai artifact."""


# ---- flatten / serialize ---------------------------------------------------------------------------------------
def flatten(artifact: dict) -> tuple[dict, dict]:
    if str(artifact.get("config", {}).get("architecture", "")) == "qwen35":
        raise ArtifactError("Qwen3.5 hybrid artifacts are a different architecture and are not supported")
    tensors = {k: np.ascontiguousarray(artifact[k]) for k in TOP_KEYS}
    for i, layer in enumerate(artifact["layers"]):
        for k in LAYER_KEYS:
            tensors[f"layers.{i}.{k}"] = np.ascontiguousarray(layer[k])
    return tensors, {"format": FORMAT, "n_layers": len(artifact["layers"]), "config": artifact["config"]}


def unflatten(tensors: dict, meta: dict) -> dict:
    art = {k: tensors[k] for k in TOP_KEYS}
    art["config"] = meta["config"]
    art["layers"] = [{k: tensors[f"layers.{i}.{k}"] for k in LAYER_KEYS} for i in range(int(meta["n_layers"]))]
    return art


def serialize(artifact: dict, provenance: dict | None = None) -> bytes:
    from safetensors.numpy import save
    tensors, meta = flatten(artifact)
    if provenance is not None:
        meta["provenance"] = provenance
    return save(tensors, metadata={"trinote": json.dumps(meta, sort_keys=True)})


def digest(artifact: dict, *, provenance: dict | None = None) -> str:
    """SHA-256 (hex) of the serialized artifact (artifact_io_bonsai.py:162-164)."""
    return hashlib.sha256(serialize(artifact, provenance)).hexdigest()


def save(artifact: dict, path, *, provenance: dict | None = None) -> str:
    """Atomic write (temp file, fsync, rename, fsync of the directory); returns the digest
    (artifact_io_bonsai.py:167-216)."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    data = serialize(artifact, provenance)
    fd, tmp = tempfile.mkstemp(prefix=f".{path.name}.", suffix=".tmp", dir=path.parent)
    try:
        with os.fdopen(fd, "wb") as f:
            f.write(data)
            f.flush()
            os.fsync(f.fileno())
        os.replace(tmp, path)
        tmp = None
        dfd = os.open(path.parent, os.O_RDONLY | getattr(os, "O_DIRECTORY", 0))
        try:
            os.fsync(dfd)
        finally:
            os.close(dfd)
    finally:
        if tmp is not None and os.path.exists(tmp):
            os.unlink(tmp)
    return hashlib.sha256(data).hexdigest()


def _sha256_file(path: Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    return h.hexdigest()


def _meta(path: Path, raw) -> dict:
    if not raw or "trinote" not in raw:
        raise ArtifactError(f"{path} is not a trinote artifact (no 'trinote' metadata)")
    try:
        meta = json.loads(raw["trinote"])
    except json.JSONDecodeError as e:
        raise ArtifactError(f"corrupt 'trinote' metadata in {path}: {e}") from e
    fmt = meta.get("format")
    if fmt == FORMAT_QWEN35:
        raise ArtifactError(f"{path}: Qwen3.5 hybrid artifacts ({FORMAT_QWEN35}) are not supported")
    if fmt != FORMAT:
        raise ArtifactError(f"not a Bonsai artifact: format {fmt!r} (need {FORMAT})")
    return meta


class _Info(dict):
    """format / provenance (/ config) eagerly; ``digest`` = SHA-256 of the file, computed on first access."""

    def __init__(self, base: dict, path: Path):
        super().__init__(base)
        self._path = path

    def __missing__(self, key):
        if key == "digest":
            d = _sha256_file(self._path)
            self[key] = d
            return d
        raise KeyError(key)


def load(path) -> tuple[dict, dict]:
    """(artifact, info) from a safetensors artifact (artifact_io_bonsai.py:246-281)."""
    from safetensors import safe_open
    path = Path(path)
    if not path.exists():
        raise ArtifactError(f"artifact not found: {path}")
    try:
        with safe_open(str(path), framework="numpy") as f:
            raw = f.metadata()
            tensors = {k: f.get_tensor(k) for k in f.keys()}
    except Exception as e:
        raise ArtifactError(f"cannot read Bonsai artifact {path}: {e}") from e
    meta = _meta(path, raw)
    try:
        art = unflatten(tensors, meta)
    except (KeyError, ValueError) as e:
        raise ArtifactError(f"Bonsai artifact {path} missing tensor {e}") from e
    return art, _Info({"format": meta["format"], "provenance": meta.get("provenance")}, path)


def read_info(path) -> dict:
    """Metadata only, no tensor reads (artifact_io_bonsai.py:284-304)."""
    from safetensors import safe_open
    path = Path(path)
    if not path.exists():
        raise ArtifactError(f"artifact not found: {path}")
    try:
        with safe_open(str(path), framework="numpy") as f:
            raw = f.metadata()
    except Exception as e:
        raise ArtifactError(f"cannot read Bonsai artifact {path}: {e}") from e
    meta = _meta(path, raw)
    return _Info({"format": meta["format"], "provenance": meta.get("provenance"), "config": meta.get("config")},
                 path)


# ---- GGUF import -----------------------------------------------------------------------------------------------
def _req_int(kv: dict, key: str) -> int:
    if key not in kv:
        raise ValueError(f"GGUF missing required key {key!r}")
    try:
        return int(kv[key])
    except (TypeError, ValueError) as e:
        raise ValueError(f"GGUF key {key!r} must be an integer, got {kv[key]!r}") from e


def _req_integral(kv: dict, key: str) -> int:
    if key not in kv:
        raise ValueError(f"GGUF missing required key {key!r}")
    try:
        f = float(kv[key])
    except (TypeError, ValueError) as e:
        raise ValueError(f"GGUF key {key!r} must be numeric, got {kv[key]!r}") from e
    if f != int(f):
        raise ValueError(f"GGUF key {key!r} must be integral, got {f}")
    return int(f)


def import_gguf(path, *, context_len: int | None = None, frac: int = 16, progress=None) -> dict:
    """Bonsai-8B Q1_0 GGUF -> artifact dict (import_bonsai_gguf.py:103-214)."""
    if not 1 <= int(frac) <= 29:
        raise ValueError(f"frac must be in [1, 29], got {frac}")
    g = _gguf.GGUF(path)
    kv = g.kv
    arch = kv.get("general.architecture", "?")
    if arch != "qwen3":
        raise ValueError(f"expected general.architecture='qwen3' for Bonsai, got {arch!r}")
    d = _req_int(kv, "qwen3.embedding_length")
    n_layers = _req_int(kv, "qwen3.block_count")
    n_heads = _req_int(kv, "qwen3.attention.head_count")
    n_kv = _req_int(kv, "qwen3.attention.head_count_kv")
    hd = int(kv.get("qwen3.attention.key_length", d // n_heads))
    if int(kv.get("qwen3.attention.value_length", hd)) != hd:
        raise ValueError(f"unsupported Bonsai value_length {kv['qwen3.attention.value_length']}; expected {hd}")
    d_ffn = _req_int(kv, "qwen3.feed_forward_length")
    base = _req_integral(kv, "qwen3.rope.freq_base")
    ctx = int(context_len or kv.get("qwen3.context_length", 65_536))
    if ctx <= 0 or ctx > MAX_CTX:
        raise ValueError(f"qwen3.context_length {ctx} out of range (1..{MAX_CTX})")
    stype = str(kv.get("qwen3.rope.scaling.type", "none"))
    factor = float(kv.get("qwen3.rope.scaling.factor", 1.0))
    orig = int(kv.get("qwen3.rope.scaling.original_context_length", ctx))
    beta_fast = float(kv.get("qwen3.rope.scaling.yarn_beta_fast", 32.0))
    beta_slow = float(kv.get("qwen3.rope.scaling.yarn_beta_slow", 1.0))
    ext = float(kv.get("qwen3.rope.scaling.yarn_ext_factor", 1.0 if stype == "yarn" else 0.0))
    attn = float(kv.get("qwen3.rope.scaling.attn_factor", 1.0))
    if progress:
        progress(f"[bonsai-import] d={d} layers={n_layers} heads={n_heads}/{n_kv} head_dim={hd} d_ffn={d_ffn} "
                 f"ctx={ctx}")
    embed_bits, embed_scale = g.q1_packed("token_embd.weight", frac)
    out_bits, out_scale = g.q1_packed("output.weight", frac)
    vocab = embed_bits.shape[0]
    if out_bits.shape[0] != vocab:
        raise ValueError(f"output vocab {out_bits.shape[0]} != embedding vocab {vocab}")
    layers = []
    for i in range(n_layers):
        layer = {k: g.fixed(f"blk.{i}.{n}.weight", frac) for k, n in _GGUF_GAIN.items()}
        for p, n in _GGUF_PROJ.items():
            layer[f"{p}_bits"], layer[f"{p}_scale_fp"] = g.q1_packed(f"blk.{i}.{n}.weight", frac)
        layers.append(layer)
    if stype == "yarn":
        cos, sin = yarn_tables(ctx, hd, base=base, freq_scale=1.0 / factor, n_ctx_orig=orig, ext_factor=ext,
                               attn_factor=attn, beta_fast=beta_fast, beta_slow=beta_slow, frac=frac)
    else:
        cos, sin = plain_tables(ctx, hd, base, frac)
    config = {"architecture": "qwen3", "dModel": d, "nLayers": n_layers, "n_heads": n_heads, "n_heads_kv": n_kv,
              "head_dim": hd, "dFfn": d_ffn, "vocab": vocab, "context_len": ctx, "frac": frac, "ropeBase": base,
              "ropeScalingType": stype, "ropeScalingFactor": factor, "ropeOriginalContextLen": orig,
              "ropeFreqScale": 1.0 / factor if factor else 1.0, "yarnExtFactor": ext, "yarnAttnFactor": attn,
              "yarnBetaFast": beta_fast, "yarnBetaSlow": beta_slow}
    return {"config": config, "embed_bits": embed_bits, "embed_scale_fp": embed_scale, "output_bits": out_bits,
            "output_scale_fp": out_scale, "final_norm_gain_fp": g.fixed("output_norm.weight", frac),
            "cos_fp": cos, "sin_fp": sin, "layers": layers}


def gguf_provenance(path, *, source: str = "prism-ml/Bonsai-8B-gguf", license: str = "Apache-2.0") -> dict:
    p = Path(path)
    return {"kind": "imported-weights", "source": source, "license": license, "ggufFile": p.name,
            "ggufSha256": _sha256_file(p), "importer": "trinote.infer_int.import_bonsai_gguf",
            "quant": "GGUF Q1_0 g128"}


# ---- device registration ---------------------------------------------------------------------------------------
def dims(artifact: dict) -> dict:
    c = artifact["config"]
    return {"n_layers": len(artifact["layers"]), "H": int(c["n_heads"]), "Hkv": int(c["n_heads_kv"]),
            "hd": int(c["head_dim"]), "d": int(c["dModel"]), "dff": int(c["dFfn"]), "vocab": int(c["vocab"]),
            "frac": int(c.get("frac", 16))}


def register_artifact(artifact: dict, *, with_head: bool = True) -> tuple[dict, dict]:
    """Upload every Q1_0 projection into the resident registry and every gain / RoPE table into the device buffer
    table; returns ``(w, g)`` handle bundles (int64 arrays per projection / gain, ``out_head``, ``finalg``,
    ``cos_h``, ``sin_h``). Raises if the device library is missing or an upload fails."""
    from . import gpu_native
    if not gpu_native.gpu_available():
        raise RuntimeError("register_artifact needs the gfx950 device library and a visible GPU")

    def q1(bits, scale):
        h = gpu_native.q1_register_weight(bits, scale)
        if h is None:
            raise RuntimeError("resident Q1_0 registration failed")
        return h

    def buf(a):
        h = gpu_native.buf_upload_i64(np.asarray(a, dtype=np.int64))
        if h is None:
            raise RuntimeError("device buffer upload failed")
        return h

    layers = artifact["layers"]
    w = {p: np.array([q1(l[f"{p}_bits"], l[f"{p}_scale_fp"]) for l in layers], dtype=np.int64) for p in PROJ}
    g = {s: np.array([buf(l[k]) for l in layers], dtype=np.int64) for s, k in GAINS.items()}
    if with_head:
        w["out_head"] = q1(artifact["output_bits"], artifact["output_scale_fp"])
        w["out_head_vocab"] = int(artifact["output_bits"].shape[0])
        g["finalg"] = buf(artifact["final_norm_gain_fp"])
    else:
        w["out_head"], w["out_head_vocab"], g["finalg"] = -1, 0, -1
    g["cos_h"] = buf(artifact["cos_fp"])
    g["sin_h"] = buf(artifact["sin_fp"])
    return w, g
