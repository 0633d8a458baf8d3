"""Bonsai artifact import / persistence (integer_inference_engine_amd/artifact.py), CPU.

Gates after bonsai/tests/test_bonsai_smoke.py:55-85 (round trip keeps the forward, the digest binds weights,
config and provenance) and import_bonsai_gguf.py:103-214 (required keys and refusals). The file layout is checked by
parsing the safetensors header directly from its published format (8-byte little-endian length, JSON header with
``dtype``/``shape``/``data_offsets`` and ``__metadata__``), not through the library the writer uses."""
import hashlib
import json
import struct

import numpy as np
import pytest

from integer_inference_engine_amd import artifact as A
from oracle import bonsai_model as obm, qk
from oracle.q1 import q1_rows
from oracle.rope import build_rope_tables, build_yarn_rope_tables
from tests.gguf_writer import artifact_model, bonsai_gguf

PROV = {"kind": "imported-weights", "source": "synthetic", "license": "test-only"}


@pytest.fixture(scope="module")
def imported(tmp_path_factory):
    p = tmp_path_factory.mktemp("g") / "bonsai.gguf"
    src = bonsai_gguf(p, seed=5)
    return p, src, A.import_gguf(p)


def test_import_matches_written_tensors(imported):
    _, src, art = imported
    c = art["config"]
    assert (c["dModel"], c["nLayers"], c["n_heads"], c["n_heads_kv"], c["head_dim"], c["dFfn"], c["vocab"],
            c["context_len"], c["ropeBase"], c["ropeScalingType"]) == (128, 2, 4, 2, 32, 256, 256, 64, 1000000, "none")
    bits, h = src["token_embd.weight"]
    assert np.array_equal(art["embed_bits"], bits)
    assert np.array_equal(art["embed_scale_fp"], qk.fp16_fixed(h, 16))
    for i, layer in enumerate(art["layers"]):
        for p, n in (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"), ("w1", "ffn_gate"),
                     ("wu", "ffn_up"), ("w2", "ffn_down")):
            bits, h = src[f"blk.{i}.{n}.weight"]
            assert np.array_equal(layer[f"{p}_bits"], bits)
            assert np.array_equal(layer[f"{p}_scale_fp"], qk.fp16_fixed(h, 16))
        g = src[f"blk.{i}.attn_k_norm.weight"].astype(np.float64)
        assert np.array_equal(layer["k_norm_gain_fp"], np.rint(g * 65536).astype(np.int64))
    cos, sin = build_rope_tables(64, 32, 1_000_000, 16)
    assert np.array_equal(art["cos_fp"], cos) and np.array_equal(art["sin_fp"], sin)


def test_import_yarn_tables(tmp_path):
    p = tmp_path / "y.gguf"
    bonsai_gguf(p, seed=6, yarn=True, n_layers=1)
    art = A.import_gguf(p)
    cos, sin = build_yarn_rope_tables(64, 32, base=1_000_000, freq_scale=0.25, n_ctx_orig=16)
    assert np.array_equal(art["cos_fp"], cos) and np.array_equal(art["sin_fp"], sin)
    assert art["config"]["ropeScalingType"] == "yarn" and art["config"]["ropeFreqScale"] == 0.25


@pytest.mark.parametrize("kw,match", [
    ({"extra_kv": [("general.architecture", "str", "llama")]}, "architecture"),
    ({"drop": ("qwen3.feed_forward_length",)}, "missing required key"),
    ({"drop": ("qwen3.rope.freq_base",), "extra_kv": [("qwen3.rope.freq_base", "f32", 10000.5)]}, "integral"),
    ({"drop": ("qwen3.context_length",), "extra_kv": [("qwen3.context_length", "u32", (1 << 20) + 1)]}, "range"),
    ({"extra_kv": [("qwen3.attention.value_length", "u32", 64)]}, "value_length"),
])
def test_import_refusals(tmp_path, kw, match):
    p = tmp_path / "r.gguf"
    if "extra_kv" in kw and kw["extra_kv"][0][0] == "general.architecture":
        kw = {"drop": ("general.architecture",), **kw}
    bonsai_gguf(p, seed=7, n_layers=1, **kw)
    with pytest.raises(ValueError, match=match):
        A.import_gguf(p)


def test_import_refuses_vocab_mismatch_and_bad_frac(tmp_path):
    p = tmp_path / "v.gguf"
    bonsai_gguf(p, seed=8, n_layers=1)
    with pytest.raises(ValueError, match="frac"):
        A.import_gguf(p, frac=30)
    bonsai_gguf(p, seed=8, n_layers=1, out_vocab=128)
    with pytest.raises(ValueError, match="vocab"):
        A.import_gguf(p)


def test_roundtrip_keeps_the_forward_and_digest_binds_identity(imported, tmp_path):
    _, _, art = imported
    p = tmp_path / "bonsai.safetensors"
    d = A.save(art, p, provenance=PROV)
    assert d == A.digest(art, provenance=PROV) == hashlib.sha256(p.read_bytes()).hexdigest()
    loaded, info = A.load(p)
    assert info["format"] == A.FORMAT and info["provenance"] == PROV and info["digest"] == d
    ri = A.read_info(p)
    assert ri["config"] == art["config"] and ri["digest"] == d
    assert A.digest(art) != d
    assert A.digest(art, provenance={**PROV, "source": "other"}) != d
    changed = {**art, "layers": [dict(l) for l in art["layers"]]}
    changed["layers"][1]["wq_scale_fp"] = art["layers"][1]["wq_scale_fp"] + 1
    assert A.digest(changed, provenance=PROV) != d
    ma, mb = artifact_model(art), artifact_model(loaded)
    ids = [1, 2, 3, 4]
    c = {"H": 4, "Hkv": 2, "hd": 32}
    xa, xb = q1_rows(*ma["embed"], ids), q1_rows(*mb["embed"], ids)
    for la, lb in zip(ma["layers"], mb["layers"]):
        xa = obm.layer_forward(xa, la, c, ma["cos"], ma["sin"], 16, None, None, 0)[0]
        xb = obm.layer_forward(xb, lb, c, mb["cos"], mb["sin"], 16, None, None, 0)[0]
    assert np.array_equal(obm.head_logits(ma, xa, 16), obm.head_logits(mb, xb, 16))


def test_safetensors_layout_from_the_published_format(imported, tmp_path):
    _, _, art = imported
    p = tmp_path / "a.safetensors"
    A.save(art, p, provenance=PROV)
    raw = p.read_bytes()
    n = struct.unpack_from("<Q", raw, 0)[0]
    hdr = json.loads(raw[8:8 + n])
    meta = json.loads(hdr.pop("__metadata__")["trinote"])
    assert meta == {"format": "trinote-artifact-bonsai-qwen3/1", "n_layers": 2, "config": art["config"],
                    "provenance": PROV}
    want_keys = set(A.TOP_KEYS) | {f"layers.{i}.{k}" for i in range(2) for k in A.LAYER_KEYS}
    assert set(hdr) == want_keys
    body = raw[8 + n:]
    for key, ent in hdr.items():
        arr = art[key] if "." not in key else art["layers"][int(key.split(".")[1])][key.split(".")[2]]
        assert ent["dtype"] == {np.dtype(np.uint8): "U8", np.dtype(np.int64): "I64"}[arr.dtype]
        assert ent["shape"] == list(arr.shape)
        s, e = ent["data_offsets"]
        assert body[s:e] == np.ascontiguousarray(arr).astype(arr.dtype.newbyteorder("<")).tobytes()


def test_load_refusals(tmp_path, imported):
    from safetensors.numpy import save_file
    with pytest.raises(A.ArtifactError, match="not found"):
        A.load(tmp_path / "missing.safetensors")
    p = tmp_path / "plain.safetensors"
    save_file({"x": np.zeros(3, np.int64)}, str(p))
    with pytest.raises(A.ArtifactError, match="no 'trinote' metadata"):
        A.load(p)
    save_file({"x": np.zeros(3, np.int64)}, str(p), metadata={"trinote": json.dumps({"format": A.FORMAT_QWEN35})})
    with pytest.raises(A.ArtifactError, match="Qwen3.5"):
        A.read_info(p)
    save_file({"x": np.zeros(3, np.int64)}, str(p), metadata={"trinote": "{"})
    with pytest.raises(A.ArtifactError, match="corrupt"):
        A.load(p)
    _, _, art = imported
    tensors, meta = A.flatten(art)
    tensors.pop("layers.1.w2_bits")
    save_file(tensors, str(p), metadata={"trinote": json.dumps(meta, sort_keys=True)})
    with pytest.raises(A.ArtifactError, match="missing tensor"):
        A.load(p)
    with pytest.raises(A.ArtifactError, match="different architecture"):
        A.flatten({"config": {"architecture": "qwen35"}})


def test_provenance_hashes_the_gguf(imported):
    p, _, _ = imported
    prov = A.gguf_provenance(p)
    assert prov["ggufSha256"] == hashlib.sha256(p.read_bytes()).hexdigest() and prov["ggufFile"] == p.name
