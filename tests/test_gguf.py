"""GGUF import (integer_inference_engine_amd/gguf.py) on files written here by an independent GGUF v3 writer (CPU).

The Q1_0 scale rule is checked against the integer restatement oracle.qk.fp16_fixed (round-half-even of
fp16 * 2^16 computed from the fp16 bits), the refusals against import_bonsai_gguf.py:69-84, and the expert slice
against the byte layout [in, out, n_experts] of north-mini-code/src/nmc/gguf.py:108-113."""
import numpy as np
import pytest

from integer_inference_engine_amd import gguf
from oracle import qk
from tests.gguf_writer import _q1_blocks, write_gguf


def test_bonsai_q1_gain_and_metadata(tmp_path):
    rng = np.random.default_rng(1)
    out_f, nb = 5, 2
    sc = np.array([0.5, -0.25, 1.0e-5, 6.0e-8, 65504.0, -3.0, 0.0, 2.0 ** -14, 0.1, -7.5], dtype=np.float16)
    blocks = _q1_blocks(rng, out_f, nb, sc)
    gain32 = rng.standard_normal(256).astype("<f4")
    gain16 = rng.standard_normal(128).astype("<f2")
    kv = [("general.architecture", "str", "qwen3"), ("qwen3.block_count", "u32", 36),
          ("qwen3.rope.freq_base", "f32", 1000000.0), ("tokenizer.ggml.tokens", "arr_str", ["a", "bc", "def"])]
    p = tmp_path / "b.gguf"
    write_gguf(p, kv, [("blk.0.attn_q.weight", [nb * 128, out_f], gguf.Q1_0, blocks.tobytes()),
                       ("blk.0.attn_norm.weight", [256], gguf.F32, gain32.tobytes()),
                       ("output_norm.weight", [128], gguf.F16, gain16.tobytes())], alignment=64)
    g = gguf.GGUF(p)
    assert g.kv["general.architecture"] == "qwen3" and g.kv["qwen3.block_count"] == 36
    assert g.kv["tokenizer.ggml.tokens"] == ["a", "bc", "def"] and g.kv["general.alignment"] == 64
    assert g.data_start % 64 == 0
    bits, scale = g.q1_packed("blk.0.attn_q.weight", 16)
    assert bits.shape == (out_f, nb, 16) and np.array_equal(bits, blocks[:, :, 2:])
    assert np.array_equal(scale, qk.fp16_fixed(sc.view(np.uint16).reshape(out_f, nb), 16))
    assert np.array_equal(g.fixed("blk.0.attn_norm.weight", 16), np.rint(gain32.astype(np.float64) * 65536).astype(np.int64))
    assert np.array_equal(g.fixed("output_norm.weight", 16), qk.fp16_fixed(gain16.view(np.uint16), 16))


@pytest.mark.parametrize("bad", [np.inf, np.nan])
def test_non_finite_scale_is_refused(tmp_path, bad):
    rng = np.random.default_rng(2)
    sc = np.array([1.0, bad], dtype=np.float16)
    p = tmp_path / "bad.gguf"
    write_gguf(p, [], [("w", [128, 2], gguf.Q1_0, _q1_blocks(rng, 2, 1, sc).tobytes())])
    with pytest.raises(ValueError, match="non-finite"):
        gguf.GGUF(p).q1_packed("w", 16)


def test_fixed_refuses_int64_overflow(tmp_path):
    p = tmp_path / "big.gguf"
    write_gguf(p, [], [("g", [2], gguf.F32, np.array([1.0, 2.0 ** 50], dtype="<f4").tobytes())])
    with pytest.raises(ValueError, match="exceeds int64"):
        gguf.GGUF(p).fixed("g", 16)


def test_nmc_expert_slices_and_rows(tmp_path):
    n_e, out_f, in_f = 3, 4, 512
    e_raw = [qk.random_blocks(7, e, out_f, in_f // 256, 0) for e in range(n_e)]
    d_raw = qk.random_blocks(8, 0, 6, in_f // 256, 1)
    p = tmp_path / "n.gguf"
    write_gguf(p, [("general.architecture", "str", "cohere2moe")],
               [("blk.1.ffn_gate_exps.weight", [in_f, out_f, n_e], gguf.Q4_K, b"".join(r.tobytes() for r in e_raw)),
                ("blk.0.attn_output.weight", [in_f, 6], gguf.Q6_K, d_raw.tobytes())])
    g = gguf.GGUF(p)
    for e in range(n_e):
        raw, of, nb, qt = g.expert_raw("blk.1.ffn_gate_exps.weight", e)
        assert (of, nb, qt) == (out_f, in_f // 256, 0)
        assert np.array_equal(np.asarray(raw), e_raw[e].reshape(-1))
        assert np.array_equal(qk.dequant(np.asarray(raw), of, nb, qt, 24), qk.dequant(e_raw[e], of, nb, qt, 24))
    raw, of, nb, qt = g.quant_rows("blk.0.attn_output.weight")
    assert (of, nb, qt) == (6, 2, 1) and np.array_equal(np.asarray(raw), d_raw.reshape(-1))
    with pytest.raises(IndexError):
        g.expert_raw("blk.1.ffn_gate_exps.weight", n_e)


def test_truncated_file_is_refused(tmp_path):
    rng = np.random.default_rng(3)
    p = tmp_path / "t.gguf"
    write_gguf(p, [], [("w", [256, 4], gguf.Q1_0, _q1_blocks(rng, 4, 2, np.ones(8, np.float16)).tobytes())])
    data = p.read_bytes()
    p.write_bytes(data[:-40])
    with pytest.raises(ValueError):
        gguf.GGUF(p)


@pytest.mark.parametrize("version,ok", [(2, True), (3, True), (1, False), (4, False)])
def test_header_versions(tmp_path, version, ok):
    p = tmp_path / "v.gguf"
    write_gguf(p, [("general.architecture", "str", "qwen3")], [("g", [4], gguf.F32, np.ones(4, "<f4").tobytes())])
    raw = bytearray(p.read_bytes())
    raw[4:8] = np.array([version], dtype="<u4").tobytes()
    p.write_bytes(bytes(raw))
    if ok:
        assert gguf.GGUF(p).version == version
    else:
        with pytest.raises(ValueError, match="version"):
            gguf.GGUF(p)


def test_unknown_value_type_and_bad_magic(tmp_path):
    import struct
    p = tmp_path / "u.gguf"
    body = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 3) + b"key" + struct.pack("<I", 99)
    p.write_bytes(body + b"\0" * 64)
    with pytest.raises(ValueError, match="value type"):
        gguf.GGUF(p)
    p.write_bytes(b"GGML" + body[4:])
    with pytest.raises(ValueError, match="not a GGUF"):
        gguf.GGUF(p)
