"""The five BASELINE configurations as seeded synthetic workloads, and their oracle outputs (test infrastructure).

Each config's inputs are pure functions of fixed seeds (oracle/prng.py streams), so a GPU run regenerates exactly
the inputs the committed golden digests (tests/golden/configs.json, written by tests/golden/make_config_golden.py)
were computed from. The oracle side uses the C restatement (oracle/c) where the numpy form would take minutes; each
C function is pinned to the numpy oracle and the reference C kernels in tests/test_oracle_c.py.

* C1 (reference_bonsai.py:149-219): Q1_0 matvec 4096x4096, codec-range int64 scales (round(fp16 * 2^16) of
  uniform finite fp16 patterns with a random sign, the importer's rule import_bonsai_gguf.py:64-93), x int8-range.
* C2 (reference_bonsai.py:941-966, 656-720): one 8B-shape layer, decode at position 4096 over a seeded cache.
* C3 (reference_bonsai.py:968-1065): the same layer shape over a 2048-token causal prefill.
* C4 (cohere2.py:162-188): MoE block, d 2048, 128 experts, top-8, expert FFN 768, 64 tokens, Q4_K/Q6_K.
* C5 (reference_bonsai.py:1175-1310): 36 layers, 32 sequences, contexts U[512, 32768], 64 greedy steps, vocab
  151,936; the cache of sequence b, layer l is the device generator's draw (workloads.kv_fill_seq, id b).
"""
from __future__ import annotations

import hashlib

import numpy as np

from . import bonsai_model as obm, c_oracle, fixedpoint as fx, prng, qk, workloads
from .q1 import argmax_lowest, q1_rows
from .rope import bonsai8b_tables

D, H, HKV, HD, DFF, VOCAB = 4096, 32, 8, 128, 12288, 151936
CFG = {"H": H, "Hkv": HKV, "hd": HD}
FRAC = 16


def sha(a: np.ndarray) -> str:
    """SHA-256 of an array's little-endian bytes (int64 as <i8)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.int64:
        a = a.astype("<i8", copy=False)
    return hashlib.sha256(a.tobytes()).hexdigest()


# ---- C1 --------------------------------------------------------------------------------------------------------
def codec_scales(seed: int, tid: int, shape) -> np.ndarray:
    h = prng.uniform_int(seed, tid, shape, 0, 0x7C00).astype(np.uint16)
    v = h.view(np.float16).astype(np.float64)
    v = np.where(prng.uniform_int(seed, tid + 1, shape, 0, 2) == 1, -v, v)
    return np.rint(v * 65536.0).astype(np.int64)


def c1_inputs(replica: int = 0):
    """Replica r of the config-1 weight (the benchmark rotates over several); replica 0 is the golden case."""
    s = 101 + replica
    bits = prng.uniform_bytes(s, 1, (D, D // 128, 16))
    scale = codec_scales(s, 2, (D, D // 128))
    x = prng.uniform_int(101, 4, (1, D), -127, 128)
    return x, bits, scale


def c1_oracle():
    x, bits, scale = c1_inputs()
    return {"out": c_oracle.q1_linear(x, bits, scale, FRAC)}


# ---- C2 / C3 ---------------------------------------------------------------------------------------------------
C2_CTX = 4096


def c2_inputs():
    layer = workloads.bonsai_layer(2, D, H, HKV, HD, DFF)
    cos, sin = bonsai8b_tables(C2_CTX + 8)
    kc, vc = workloads.kv_fill(2, 50, HKV, C2_CTX, HD)
    x = prng.uniform_int(2, 60, (1, D), -(1 << 20), 1 << 20)
    return layer, cos, sin, kc, vc, x


def c2_oracle():
    layer, cos, sin, kc, vc, x = c2_inputs()
    out, kn, vn = obm.layer_forward(x, layer, CFG, cos, sin, FRAC, kc, vc, C2_CTX, q1=c_oracle.q1_linear,
                                    attn=c_oracle.attention_cached, silu_mul=c_oracle.silu_mul)
    return {"out": out, "k_new": kn, "v_new": vn}


C3_T = 2048


def c3_inputs(T: int = C3_T):
    layer = workloads.bonsai_layer(3, D, H, HKV, HD, DFF)
    cos, sin = bonsai8b_tables(T + 64)
    x = prng.uniform_int(3, 60, (T, D), -(1 << 20), 1 << 20)
    return layer, cos, sin, x


def c3_oracle(T: int = C3_T):
    layer, cos, sin, x = c3_inputs(T)
    out, k, v = obm.layer_forward(x, layer, CFG, cos, sin, FRAC, None, None, 0, q1=c_oracle.q1_linear,
                                  attn=c_oracle.attention_cached, silu_mul=c_oracle.silu_mul)
    return {"out": out, "k": k, "v": v}


# ---- C4 --------------------------------------------------------------------------------------------------------
C4 = dict(seed=4, E=128, k=8, d=2048, e_ffn=768, T=64)


def c4_experts(seed: int, E: int, d: int, e_ffn: int):
    return [dict(gate=qk.random_blocks(seed, 100 + 3 * e, e_ffn, d // 256, 0),
                 up=qk.random_blocks(seed, 101 + 3 * e, e_ffn, d // 256, 0),
                 down=qk.random_blocks(seed, 102 + 3 * e, d, e_ffn // 256, 1)) for e in range(E)]


def c4_inputs(seed=C4["seed"], E=C4["E"], k=C4["k"], d=C4["d"], e_ffn=C4["e_ffn"], T=C4["T"]):
    ex = c4_experts(seed, E, d, e_ffn)
    h = prng.uniform_int(seed, 7, (T, d), -(1 << 16), 1 << 16)
    logits = prng.uniform_int(seed, 8, (T, E), -(1 << 20), 1 << 20)
    sel, gates = qk.moe_route(logits, k, FRAC)
    return ex, h, sel, gates


def c4_oracle():
    d, e_ffn = C4["d"], C4["e_ffn"]
    ex, h, sel, gates = c4_inputs()
    used = sorted(set(int(e) for e in sel.reshape(-1)))
    raw = {e: dict(gate=(ex[e]["gate"], e_ffn, d // 256, 0), up=(ex[e]["up"], e_ffn, d // 256, 0),
                   down=(ex[e]["down"], d, e_ffn // 256, 1)) for e in used}
    lin = lambda x, w, fw: c_oracle.qk_linear(w[0], x, w[1], w[2], fw, w[3])
    return {"out": qk.moe_ffn_grouped(h, sel, gates, raw, FRAC, 24, lin), "sel": sel, "gates": gates}


# ---- C5 --------------------------------------------------------------------------------------------------------
C5 = dict(seed=13, B=32, steps=64, n_layers=36, lo=512, hi=32768)


def c5_spec():
    """(lens, first tokens, rope rows needed) of the config-5 batch."""
    s = C5["seed"]
    lens = prng.uniform_int(s, 1, (C5["B"],), C5["lo"], C5["hi"] + 1)
    first = prng.uniform_int(s, 2, (C5["B"],), 0, VOCAB)
    return lens, first, int(lens.max()) + C5["steps"] + 8


def c5_model(n_layers: int = C5["n_layers"]):
    s = C5["seed"]
    _, _, ctx = c5_spec()
    cos, sin = bonsai8b_tables(ctx)
    return {"layers": [workloads.bonsai_layer(s, D, H, HKV, HD, DFF, li) for li in range(n_layers)],
            "cos": cos, "sin": sin, "embed": workloads.q1_weight(s, 7, VOCAB, D),
            "out": workloads.q1_weight(s, 9, VOCAB, D),
            "final_g": prng.uniform_int(s, 11, (D,), 1 << 15, (1 << 17) + 1)}


def c5_buffers(n_layers: int = C5["n_layers"]):
    """Per-layer K/V row buffers (Hkv, cap, hd) int64 sized for the longest sequence, reused across sequences."""
    _, _, ctx = c5_spec()
    return [(np.empty((HKV, ctx, HD), dtype=np.int64), np.empty((HKV, ctx, HD), dtype=np.int64))
            for _ in range(n_layers)]


def c5_sequence(model, b: int, steps: int, bufs=None, log=None):
    """Greedy decode of sequence b alone (rows of a batched decode are independent, reference_bonsai.py:1175-1199):
    its cache holds lens[b] positions of the device generator's draw for every layer; returns (tokens (steps,),
    per-step SHA-256 of the logits row). ``bufs`` (c5_buffers) are overwritten."""
    lens, first, _ = c5_spec()
    L0 = int(lens[b])
    bufs = bufs if bufs is not None else c5_buffers(len(model["layers"]))
    for li, pair in enumerate(bufs[:len(model["layers"])]):
        assert pair[0].shape[1] >= L0 + steps
        for kind, buf in enumerate(pair):
            # element (kv, j, c) of the (Hkv, L0, hd) draw has index (kv * L0 + j) * hd + c
            tid = 100000 + 1024 * li + 512 * kind + b
            for kv in range(HKV):
                c_oracle.uniform_fill(C5["seed"], tid, buf[kv], L0, HD, -(1 << 20), 1 << 20, first=kv * L0 * HD)
    tok = int(first[b])
    toks, digs = [], []
    for s in range(steps):
        x = q1_rows(*model["embed"], np.array([tok]))
        for li, layer in enumerate(model["layers"]):
            kb, vb = bufs[li]
            x = obm.layer_forward_rowbuf(x, layer, CFG, model["cos"], model["sin"], FRAC, kb, vb, L0 + s,
                                         q1=c_oracle.q1_linear, silu_mul=c_oracle.silu_mul)
        lg = c_oracle.q1_linear(fx.rmsnorm(x, FRAC, 1, model["final_g"]), *model["out"], FRAC)[0]
        tok = int(argmax_lowest(lg[None])[0])
        toks.append(tok)
        digs.append(sha(lg))
        if log:
            log(f"seq {b} step {s} token {tok}")
    return toks, digs


def c5_step_digest(row_digests) -> str:
    """Digest of one step over the batch: SHA-256 of the concatenated per-sequence row digests (hex), in order."""
    return hashlib.sha256("".join(row_digests).encode()).hexdigest()
