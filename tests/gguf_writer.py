"""A small GGUF v3 writer for tests (written from the published GGUF layout: magic, version, counts, typed KV
pairs, tensor infos, aligned data section), independent of the reader under test."""
import struct

import numpy as np


def _s(b: bytes) -> bytes:
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, kv, tensors, alignment=32):
    """kv: [(key, kind, value)] with kind 'u32' / 'f32' / 'str' / 'arr_str'; tensors: [(name, shape, type, bytes)]."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv) + 1))
    for key, kind, val in kv + [("general.alignment", "u32", alignment)]:
        out += _s(key.encode())
        if kind == "u32":
            out += struct.pack("<II", 4, val)
        elif kind == "f32":
            out += struct.pack("<If", 6, val)
        elif kind == "str":
            out += struct.pack("<I", 8) + _s(val.encode())
        elif kind == "arr_str":
            out += struct.pack("<IIQ", 9, 8, len(val)) + b"".join(_s(v.encode()) for v in val)
    offs, off = [], 0
    for name, shape, tt, data in tensors:
        offs.append(off)
        out += _s(name.encode()) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", tt, off)
        off = (off + len(data) + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    base = len(out)
    for (_, _, _, data), o in zip(tensors, offs):
        assert len(out) - base == o
        out += data + b"\0" * ((-len(data)) % alignment)
    path.write_bytes(bytes(out))


def _q1_blocks(rng, out_f, nb, scales_f16):
    blocks = np.zeros((out_f, nb, 18), dtype=np.uint8)
    blocks[:, :, :2] = scales_f16.reshape(out_f, nb).astype("<f2").view(np.uint8).reshape(out_f, nb, 2)
    blocks[:, :, 2:] = rng.integers(0, 256, size=(out_f, nb, 16), dtype=np.uint8)
    return blocks


def bonsai_gguf(path, seed: int = 0, *, d=128, H=4, Hkv=2, hd=32, dff=256, n_layers=2, vocab=256, ctx=64,
                yarn=False, extra_kv=(), drop=(), out_vocab=None):
    """A small Bonsai (qwen3, Q1_0) GGUF with random fp16 scales and F32 gains; returns the written source data
    {tensor name: (bits, fp16 scales) | f32 gain}."""
    rng = np.random.default_rng(seed)
    kv = [("general.architecture", "str", "qwen3"), ("qwen3.embedding_length", "u32", d),
          ("qwen3.block_count", "u32", n_layers), ("qwen3.attention.head_count", "u32", H),
          ("qwen3.attention.head_count_kv", "u32", Hkv), ("qwen3.attention.key_length", "u32", hd),
          ("qwen3.feed_forward_length", "u32", dff), ("qwen3.rope.freq_base", "f32", 1000000.0),
          ("qwen3.context_length", "u32", ctx)]
    if yarn:
        kv += [("qwen3.rope.scaling.type", "str", "yarn"), ("qwen3.rope.scaling.factor", "f32", 4.0),
               ("qwen3.rope.scaling.original_context_length", "u32", 16)]
    kv = [e for e in kv if e[0] not in drop] + list(extra_kv)
    src, tensors = {}, []

    def q1(name, out_f, in_f):
        sc = (rng.uniform(0.002, 0.03, size=out_f * (in_f // 128)) * rng.choice([-1, 1], out_f * (in_f // 128)))
        blocks = _q1_blocks(rng, out_f, in_f // 128, sc.astype(np.float16))
        src[name] = (blocks[:, :, 2:].copy(), blocks[:, :, :2].copy().view("<u2").reshape(out_f, in_f // 128))
        tensors.append((name, [in_f, out_f], 41, blocks.tobytes()))

    def gain(name, n):
        g = rng.uniform(0.5, 2.0, size=n).astype("<f4")
        src[name] = g
        tensors.append((name, [n], 0, g.tobytes()))

    q1("token_embd.weight", vocab, d)
    q1("output.weight", out_vocab or vocab, d)
    gain("output_norm.weight", d)
    shapes = {"attn_q": (H * hd, d), "attn_k": (Hkv * hd, d), "attn_v": (Hkv * hd, d), "attn_output": (d, H * hd),
              "ffn_gate": (dff, d), "ffn_up": (dff, d), "ffn_down": (d, dff)}
    for i in range(n_layers):
        for n, (o, k) in shapes.items():
            q1(f"blk.{i}.{n}.weight", o, k)
        for n, size in (("attn_norm", d), ("ffn_norm", d), ("attn_q_norm", hd), ("attn_k_norm", hd)):
            gain(f"blk.{i}.{n}.weight", size)
    write_gguf(path, kv, [t for t in tensors if t[0] not in drop])
    return src


def artifact_model(art) -> dict:
    """An artifact dict in the oracle model layout (oracle.bonsai_model)."""
    c = art["config"]
    layers = []
    for l in art["layers"]:
        m = {p: (l[f"{p}_bits"], l[f"{p}_scale_fp"]) for p in ("wq", "wk", "wv", "wo", "w1", "wu", "w2")}
        m.update(n1g=l["n1_gain_fp"], n2g=l["n2_gain_fp"], qng=l["q_norm_gain_fp"], kng=l["k_norm_gain_fp"])
        layers.append(m)
    return {"cfg": {"d": c["dModel"], "H": c["n_heads"], "Hkv": c["n_heads_kv"], "hd": c["head_dim"],
                    "dff": c["dFfn"], "n_layers": c["nLayers"], "vocab": c["vocab"], "frac": c["frac"]},
            "layers": layers, "cos": art["cos_fp"], "sin": art["sin_fp"],
            "embed": (art["embed_bits"], art["embed_scale_fp"]), "out": (art["output_bits"], art["output_scale_fp"]),
            "final_g": art["final_norm_gain_fp"]}
