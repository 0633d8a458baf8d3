#!/usr/bin/env python3
"""Benchmark of the hot path on one MI355X: packed Q1_0 matvec HBM GB/s (BASELINE.json metric, config 1).

One step = one launch of the Q1_0 matvec over a rotation of R distinct 4096x4096 weight replicas (R=384,
~1.2 GB of resident weights, so the working set cannot live in the 256 MB Infinity Cache) against one int8-range
activation vector, all inputs already resident in HBM. Scales are codec-range (round(fp16 * 2^16) of random
finite fp16 values), which do not fit int32, so the resident layout keeps 8-byte scales.

Prints ONE JSON line (driver contract) with ``roofline`` (dominant kernel timed with HIP events on its own
stream) and ``cpu_baseline`` (the reference's C kernel ``bonsai_q1_linear_i64`` compiled from its sources into
oracle/_ref, timed on this host's cores on a bounded sample).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
HBM_PEAK_GBS = 8000.0
K = 4096
NB = K // 128


def codec_scales(rng, shape):
    """round_half_even(v * 2^16) for v uniform over finite fp16 bit patterns with a random sign."""
    h = rng.integers(0, 0x7C00, size=shape, dtype=np.uint16)
    v = h.view(np.float16).astype(np.float64)
    v = np.where(rng.integers(0, 2, size=shape) == 1, -v, v)
    return np.rint(v * 65536.0).astype(np.int64)


def matvec_bytes(scale_bytes: int) -> int:
    """Algorithmic HBM bytes of one 4096x4096 Q1_0 matvec: bits + scales + x + y."""
    return K * NB * 16 + K * NB * scale_bytes + K * 8 + K * 8


def _ref_q1(port: bool = False):
    """(function, kind) of the CPU Q1 linear: the reference's C kernel built from its sources into oracle/_ref when
    present ("reference"), else (or with port=True) the C restatement of the oracle ("port")."""
    ref = ROOT / "oracle" / "_ref" / "libbonsai_q1_kernel.so"
    if ref.exists() and not port:
        so = ctypes.CDLL(str(ref))
        fn, kind = so.bonsai_q1_linear_i64, "reference"
    else:
        from oracle import c_oracle
        fn, kind = c_oracle.lib().imo_q1_linear, "port"
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 4 + [ctypes.c_void_p]
    return fn, kind


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it, with the family / model / stepping numbers (a virtualized host may
    report only a generic model name)."""
    info = {}
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if ":" in line:
                k, v = (t.strip() for t in line.split(":", 1))
                info.setdefault(k, v)
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    ids = ", ".join(f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info)
    extra = ", ".join(x for x in (ids, f"{info['cache size']} cache" if "cache size" in info else "") if x)
    return f"{name} ({extra})" if extra else name


def cpu_worker(npz: str, seconds: float, reps: int, port: bool = False) -> None:
    """Time the CPU Q1 linear on the config-1 matvec: ``reps`` repetitions of ``seconds`` each with the thread
    count this process was given (OMP_NUM_THREADS); print one JSON line with the median."""
    d = np.load(npz)
    x, bits, scale, gpu_out = d["x"], d["bits"], d["scale"], d["out"]
    fn, kind = _ref_q1(port)
    out = np.empty((1, K), dtype=np.int64)
    call = lambda: fn(x.ctypes.data, bits.ctypes.data, scale.ctypes.data, 1, K, NB, 16, out.ctypes.data)
    assert call() == 0
    match = bool(np.array_equal(out, gpu_out))
    rates, calls = [], 0
    for _ in range(reps):
        n, t0 = 0, time.perf_counter()
        while True:
            call()
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        rates.append(matvec_bytes(8) * n / el / 1e9)
        calls += n
    print(json.dumps({"value": float(np.median(rates)), "reps": rates, "unit": "GB/s", "kind": kind,
                      "calls": calls, "seconds": seconds * reps, "match": match}))


def decode_leg(so, torch, tokens: int, ctx: int = 4096, n_layers: int = 36, vocab: int = 151936,
               c5_tokens: int = 0) -> dict:
    """Bonsai-8B-shape greedy decode at batch 1: embed -> 36 layers over a paged int32 KV cache holding ``ctx``
    positions -> final RMSNorm + Q1_0 LM head (151936x4096) -> lowest-index argmax -> next embed, all on device.

    Weights are seeded random Q1_0 of the 8B shapes; the 36 layers are 36 separately resident copies of one
    random layer (the HBM traffic per token is that of 36 distinct layers). The timed loop is ``tokens`` decode
    steps back to back on one stream with no host synchronisation. Byte-exactness of this path against the
    oracle is what tests/test_gpu_decode_8b.py checks."""
    from integer_inference_engine_amd import gpu_native as gn
    from integer_inference_engine_amd.resident import ResidentNet
    from integer_inference_engine_amd.rope_tables import bonsai8b_tables
    d, H, Hkv, hd, dff = 4096, 32, 8, 128, 12288
    rng = np.random.default_rng(8)
    shapes = {"wq": (H * hd, d), "wk": (Hkv * hd, d), "wv": (Hkv * hd, d), "wo": (d, H * hd),
              "w1": (dff, d), "wu": (dff, d), "w2": (d, dff)}
    layer = {k: (rng.integers(0, 256, size=(o, i // 128, 16), dtype=np.uint8),
                 rng.integers(1, 4097, size=(o, i // 128), dtype=np.int64)) for k, (o, i) in shapes.items()}
    gains = {k: rng.integers(1 << 15, (1 << 17) + 1, size=(n,), dtype=np.int64)
             for k, n in (("n1g", d), ("n2g", d), ("qng", hd), ("kng", hd))}
    w = {k: np.array([gn.q1_register_weight(*layer[k]) for _ in range(n_layers)], dtype=np.int64) for k in shapes}
    g = {k: np.array([gn.buf_upload_i64(v) for _ in range(n_layers)], dtype=np.int64) for k, v in gains.items()}
    assert all((v >= 0).all() for v in list(w.values()) + list(g.values())), _lib_err()
    hbits = rng.integers(0, 256, size=(vocab, d // 128, 16), dtype=np.uint8)
    hscale = rng.integers(1, 4097, size=(vocab, d // 128), dtype=np.int64)
    w["out_head"], w["out_head_vocab"] = gn.q1_register_weight(hbits, hscale), vocab
    g["finalg"] = gn.buf_upload_i64(rng.integers(1 << 15, (1 << 17) + 1, size=(d,), dtype=np.int64))
    if tokens <= 0:                                   # config 5 alone (profiling it without the b=1 leg's kernels)
        ebits = torch.from_numpy(hbits).cuda()
        escale = torch.from_numpy(hscale).cuda()
        return {"_c5": c5_leg(so, torch, w, g, ebits, escale, c5_tokens) if c5_tokens > 0 else None}
    cap = ctx + tokens + 2 + 8 + 4 + 64
    cos, sin = bonsai8b_tables(cap)
    g["cos_h"], g["sin_h"] = gn.buf_upload_i64(cos), gn.buf_upload_i64(sin)
    net = ResidentNet(B=1, n_layers=n_layers, H=H, Hkv=Hkv, hd=hd, d=d, dff=dff, cap=cap, w=w, g=g, page=64,
                      kv32=True)
    k1 = rng.integers(-(1 << 20), 1 << 20, size=(Hkv, ctx, hd), dtype=np.int64)
    v1 = rng.integers(-(1 << 20), 1 << 20, size=(Hkv, ctx, hd), dtype=np.int64)
    net.seed(0, np.broadcast_to(k1, (n_layers,) + k1.shape), np.broadcast_to(v1, (n_layers,) + v1.shape))
    del k1, v1
    ebits = torch.from_numpy(hbits).cuda()
    escale = torch.from_numpy(hscale).cuda()
    ids = torch.tensor([7], dtype=torch.int64, device="cuda")
    logits = torch.empty((1, vocab), dtype=torch.int64, device="cuda")
    hist = torch.empty((tokens, 1), dtype=torch.int64, device="cuda")
    sp = ctypes.c_void_p(net.stream.cuda_stream)
    so.imie_net_status(net.h, 1, sp)

    def run(n, graph):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        net.stream.synchronize()
        e0.record(net.stream)
        t0 = time.perf_counter()
        net.decode(ebits, escale, ids, n, graph=graph, hist=hist[:n], logits=logits)
        e1.record(net.stream)
        th = time.perf_counter() - t0
        net.stream.synchronize()
        return e0.elapsed_time(e1), th

    run(2, True)                                  # warm-up: sizes the workspaces and captures the step graph
    ms_eager, _ = run(min(tokens, 8), False)
    ms_eager /= min(tokens, 8)
    ms, t_host = run(tokens, True)                # timed: one call, step 1 eager + (tokens - 1) graph replays
    # per-kernel-family split from a separate eager profiled pass (the profiler's events add host work)
    prof = {}
    so.imie_profile_begin()
    run(4, False)
    for kid, name in ((0, "q1_prep"), (1, "q1_gemv"), (3, "attention")):
        kms, kcnt = ctypes.c_double(), ctypes.c_int64()
        so.imie_profile_read(kid, ctypes.byref(kms), ctypes.byref(kcnt))
        prof[name + "_ms_per_token"] = round(kms.value / 4, 4)
    so.imie_profile_end()
    status = int(so.imie_net_status(net.h, 0, sp))
    last = int(ids.item())
    net.close()
    c5 = c5_leg(so, torch, w, g, ebits, escale, c5_tokens) if c5_tokens > 0 else None
    wbytes = sum(o * (i // 128) * (16 + 4) for o, i in shapes.values()) * n_layers + vocab * (d // 128) * 20
    kvbytes = n_layers * 2 * Hkv * ctx * hd * 4
    return {"tok_s": round(tokens / (ms / 1e3), 2), "ms_per_token": round(ms / tokens, 3),
            "host_enqueue_ms_per_token": round(t_host * 1e3 / tokens, 3), "eager_ms_per_token": round(ms_eager, 3),
            "mode": "HIP graph of one greedy step (embed, 36 layers, head, argmax), replayed", "tokens": tokens,
            "context": ctx,
            "layers": n_layers, "vocab": vocab, "kv": "kv8 digit planes (int8 x 4 per element), 64-slot pages", "status": status,
            "last_token": last, "weight_plus_kv_GB_per_token": round((wbytes + kvbytes) / 1e9, 3),
            "effective_GB_s": round((wbytes + kvbytes) / (ms / tokens / 1e3) / 1e9, 1), **prof, "_c5": c5}


def c5_leg(so, torch, w, g, ebits, escale, tokens: int, B: int = 32, n_layers: int = 36) -> dict:
    """Config 5: the 36-layer 8B-shape stack (same resident weights as the b=1 leg) decoding a ragged batch of B
    sequences with contexts drawn uniformly from [512, 32768] over a paged kv8 cache (device-generated seeded
    contents, ~153 GB), `tokens` greedy tokens each, as one device call replaying a HIP graph per step."""
    from integer_inference_engine_amd.resident import ResidentNet
    from integer_inference_engine_amd.rope_tables import bonsai8b_tables
    d, H, Hkv, hd, dff = 4096, 32, 8, 128, 12288
    rng = np.random.default_rng(55)
    lens = rng.integers(512, 32769, size=B).astype(np.int64)
    extra = 2 * tokens + 8                             # greedy warm-up + timed run, then the sampled run
    cap = int(lens.max()) + extra
    cos, sin = bonsai8b_tables(cap)
    from integer_inference_engine_amd import gpu_native as gn
    g = dict(g)
    g["cos_h"], g["sin_h"] = gn.buf_upload_i64(cos), gn.buf_upload_i64(sin)
    net = ResidentNet(B=B, n_layers=n_layers, H=H, Hkv=Hkv, hd=hd, d=d, dff=dff, cap=64, w=w, g=g, page=64,
                      kv32=True)
    t0 = time.perf_counter()
    net.set_caps(lens + extra)
    net.fill_kv(55, lens)
    setup_s = time.perf_counter() - t0
    ids = torch.tensor(rng.integers(0, ebits.shape[0], size=B), dtype=torch.int64, device="cuda")
    logits = torch.empty((B, ebits.shape[0]), dtype=torch.int64, device="cuda")
    hist = torch.empty((tokens, B), dtype=torch.int64, device="cuda")
    net.clear_status()
    net.decode(ebits, escale, ids, 2, graph=True, hist=hist[:2], logits=logits)      # warm-up + graph capture
    net.stream.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(net.stream)
    net.decode(ebits, escale, ids, tokens, graph=True, hist=hist, logits=logits)
    e1.record(net.stream)
    net.stream.synchronize()
    ms = e0.elapsed_time(e1)
    status = net.status()
    # the same step with the device sampler instead of argmax (qwen3-rec preset: T 0.6, top-k 20, top-p 0.95),
    # histories = the greedy tokens so far; tokens - 2 timed steps after one eager + one captured step
    from types import SimpleNamespace
    scfg = SimpleNamespace(mode="top_p", temperature=0.6, top_k=20, top_p=0.95, min_p=0.0, seed=0, rep_penalty=0,
                           no_repeat_ngram=0)
    hld = 2 * tokens + 8
    shist = torch.full((B, hld), -1, dtype=torch.int64, device="cuda")
    shist[:, :tokens] = hist.t()
    slen = torch.full((B,), tokens, dtype=torch.int64, device="cuda")
    net.decode_sampled(ebits, escale, ids, 2, scfg, 16, shist, slen, graph=True, logits=logits)
    net.stream.synchronize()
    ns = max(tokens - 2, 1)
    e0.record(net.stream)
    net.decode_sampled(ebits, escale, ids, ns, scfg, 16, shist, slen, graph=True, logits=logits)
    e1.record(net.stream)
    net.stream.synchronize()
    ms_s = e0.elapsed_time(e1)
    status |= net.status()
    net.close()
    kv_bytes = int((lens + 2).sum()) * n_layers * 2 * Hkv * hd * 4
    return {"sequences": B, "tokens_per_sequence": tokens, "layers": n_layers,
            "context_min": int(lens.min()), "context_max": int(lens.max()), "context_mean": round(float(lens.mean()), 1),
            "tok_s": round(B * tokens / (ms / 1e3), 1), "ms_per_step": round(ms / tokens, 3), "status": status,
            "kv_GB": round(kv_bytes / 1e9, 1), "kv_read_GB_s": round(kv_bytes / (ms / tokens / 1e3) / 1e9, 1),
            "setup_s": round(setup_s, 2), "kv": "kv8 digit planes (int8 x 4 per element), 64-slot pages",
            "sampled_tok_s": round(B * ns / (ms_s / 1e3), 1), "sampled_ms_per_step": round(ms_s / ns, 3),
            "sampled_mode": "top_p, qwen3-rec (T 0.6, top-k 20, top-p 0.95), device SHA-256 draws"}


def prefill_leg(so, torch, T: int = 2048) -> dict:
    """Config 3: one Bonsai-8B-shape decoder layer in prefill over a T-token prompt (causal attention over all T
    positions, int32 paged KV). Seeded random Q1_0 weights and activations; timed on one stream with HIP events.
    The Q1 projections run as int8-MFMA GEMMs (tokens in M); `q1_gemm_alg_TOPS` counts 2*T*N*K ops of the
    projections over the GEMM kernels' time (each +-1 weight times an int64 activation counted as one MAC);
    `q1_gemm_mfma_util` counts the int8 MFMA ops the kernels executed (one MAC per limb)."""
    from integer_inference_engine_amd import gpu_native as gn
    from integer_inference_engine_amd.resident import ResidentNet
    from integer_inference_engine_amd.rope_tables import bonsai8b_tables
    d, H, Hkv, hd, dff = 4096, 32, 8, 128, 12288
    rng = np.random.default_rng(3)
    shapes = {"wq": (H * hd, d), "wk": (Hkv * hd, d), "wv": (Hkv * hd, d), "wo": (d, H * hd),
              "w1": (dff, d), "wu": (dff, d), "w2": (d, dff)}
    w = {k: np.array([gn.q1_register_weight(rng.integers(0, 256, size=(o, i // 128, 16), dtype=np.uint8),
                                            rng.integers(1, 4097, size=(o, i // 128), dtype=np.int64))],
                     dtype=np.int64) for k, (o, i) in shapes.items()}
    g = {k: np.array([gn.buf_upload_i64(rng.integers(1 << 15, (1 << 17) + 1, size=(n,), dtype=np.int64))],
                     dtype=np.int64) for k, n in (("n1g", d), ("n2g", d), ("qng", hd), ("kng", hd))}
    w["out_head"], w["out_head_vocab"], g["finalg"] = -1, 0, -1
    cos, sin = bonsai8b_tables(T + 64)
    g["cos_h"], g["sin_h"] = gn.buf_upload_i64(cos), gn.buf_upload_i64(sin)
    net = ResidentNet(B=1, n_layers=1, H=H, Hkv=Hkv, hd=hd, d=d, dff=dff, cap=T + 64, w=w, g=g, page=64, kv32=True)
    x0 = torch.from_numpy(rng.integers(-(1 << 20), 1 << 20, size=(T, d), dtype=np.int64)).cuda()
    x = torch.empty_like(x0)
    torch.cuda.set_stream(net.stream)
    x.copy_(x0)
    st = net.forward(x, [0], T)                    # warm-up (sizes workspaces)
    # further untimed forwards for at least 0.25 s, so the timed ones run at the device's sustained clocks
    t_end = time.perf_counter() + 0.25
    while time.perf_counter() < t_end:
        x.copy_(x0)
        net.forward(x, [0], T)
        net.stream.synchronize()
    reps = 5
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    net.stream.synchronize()
    gops = ctypes.c_ulonglong()
    so.imie_profile_gemm_ops(ctypes.byref(gops), 1)
    so.imie_profile_begin()
    for e0, e1 in ev:                               # the input copy between forwards is outside the timed spans
        x.copy_(x0)
        e0.record(net.stream)
        st = net.forward(x, [0], T)
        e1.record(net.stream)
    net.stream.synchronize()
    ms = sum(e0.elapsed_time(e1) for e0, e1 in ev) / reps
    so.imie_profile_gemm_ops(ctypes.byref(gops), 1)
    gops.value //= reps
    prof = {}
    for kid, name in ((0, "q1_prep"), (2, "q1_gemm"), (3, "attention")):
        kms, kcnt = ctypes.c_double(), ctypes.c_int64()
        so.imie_profile_read(kid, ctypes.byref(kms), ctypes.byref(kcnt))
        prof[name + "_ms"] = round(kms.value / reps, 3)
    so.imie_profile_end()
    net.close()
    so.bonsai_q1_free_weights()
    ops = 2 * T * sum(o * i for o, i in shapes.values())
    gemm_ms = prof["q1_gemm_ms"]
    peak = ctypes.c_double()                          # measured sustained int8 MFMA ops/s of this device
    mpeak = peak.value if so.imie_mfma_peak(ctypes.byref(peak)) == 0 and peak.value > 0 else None
    return {"tokens": T, "layer_ms": round(ms, 3), "tok_s": round(T / (ms / 1e3), 1), "status": int(st),
            "q1_gemm_alg_TOPS": round(ops / (gemm_ms / 1e3) / 1e12, 1) if gemm_ms > 0 else None,
            "q1_gemm_frac_of_int8_peak": round(ops / (gemm_ms / 1e3) / 5.0e15, 4) if gemm_ms > 0 else None,
            # executed int8 MFMA ops (2*M*N*K per limb the kernels ran, counted on the device from the limb
            # tables, padding tiles included) over the GEMM kernels' time: utilisation of the 5.0 POPS peak
            "q1_gemm_mfma_ops": int(gops.value), "q1_gemm_mean_limbs": round(gops.value / ops, 3) if ops else None,
            "q1_gemm_mfma_util": round(gops.value / (gemm_ms / 1e3) / 5.0e15, 4) if gemm_ms > 0 else None,
            # the same against the measured sustained MFMA throughput (imie_mfma_peak), when that is lower
            "int8_mfma_measured_peak_POPS": round(mpeak / 1e15, 3) if mpeak else None,
            "q1_gemm_mfma_util_measured_peak": (round(gops.value / (gemm_ms / 1e3) / mpeak, 4)
                                                if mpeak and gemm_ms > 0 else None), **prof}


def moe_leg(so, torch, E: int = 128, k: int = 8, d: int = 2048, e_ffn: int = 768, T: int = 64) -> dict:
    """Config 4: north-mini-code MoE FFN block, hidden 2048, 128 experts top-8, expert FFN 768; gate/up Q4_K and
    down Q6_K raw GGML blocks (seeded random quants, finite fp16 scales), 64 tokens routed by seeded integer
    logits (ragged per-expert groups). Timed on one stream with HIP events; bytes = the distinct experts' blocks."""
    from integer_inference_engine_amd import qk_gpu
    rng = np.random.default_rng(4)

    def blocks(out_f, nb, qtype):
        bs = 144 if qtype == 0 else 210
        raw = rng.integers(0, 256, size=(out_f * nb, bs), dtype=np.uint8)
        dv = rng.uniform(0.002, 0.01, size=out_f * nb).astype(np.float16).view(np.uint16)
        if qtype == 0:
            mv = rng.uniform(0.0, 0.005, size=out_f * nb).astype(np.float16).view(np.uint16)
            raw[:, 0], raw[:, 1], raw[:, 2], raw[:, 3] = dv & 0xFF, dv >> 8, mv & 0xFF, mv >> 8
        else:
            raw[:, 208], raw[:, 209] = dv & 0xFF, dv >> 8
        return raw.reshape(-1)

    hs = []
    for _ in range(E):
        hs.append((qk_gpu.register_weight(blocks(e_ffn, d // 256, 0), e_ffn, d // 256, 0),
                   qk_gpu.register_weight(blocks(e_ffn, d // 256, 0), e_ffn, d // 256, 0),
                   qk_gpu.register_weight(blocks(d, e_ffn // 256, 1), d, e_ffn // 256, 1)))
    logits = rng.integers(-(1 << 20), 1 << 20, size=(T, E))
    sel = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    gates = rng.integers(1, 1 << 16, size=(T, k)).astype(np.int64)
    flat = sel.reshape(-1)
    arr = lambda i: (ctypes.c_int64 * (T * k))(*[hs[e][i] for e in flat])
    ga, ua, da = arr(0), arr(1), arr(2)
    h = torch.from_numpy(rng.integers(-(1 << 16), 1 << 16, size=(T, d), dtype=np.int64)).cuda()
    gd = torch.from_numpy(np.ascontiguousarray(gates.reshape(-1))).cuda()
    out = torch.empty((T, d), dtype=torch.int64, device="cuda")
    st = torch.cuda.Stream()
    sp = ctypes.c_void_p(st.cuda_stream)
    call = lambda: so.imie_moe_ffn_batched_dev(ga, ua, da, T, k, ctypes.c_void_p(h.data_ptr()),
                                               ctypes.c_void_p(gd.data_ptr()), d, e_ffn, 16, 24,
                                               ctypes.c_void_p(out.data_ptr()), sp)
    so.imie_moe_status(1, sp)
    assert call() == 0
    st.synchronize()
    t_end = time.perf_counter() + 0.25                 # untimed calls: the timed ones run at sustained clocks
    while time.perf_counter() < t_end:
        call()
        st.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 5
    e0.record(st)
    for _ in range(reps):
        call()
    e1.record(st)
    st.synchronize()
    ms = e0.elapsed_time(e1) / reps
    status = so.imie_moe_status(0, sp)
    qk_gpu.free_all()
    used = len(set(flat.tolist()))
    nbytes = used * (2 * e_ffn * (d // 256) * 144 + d * (e_ffn // 256) * 210)
    return {"tokens": T, "experts": E, "top_k": k, "experts_used": used, "ms": round(ms, 3),
            "tok_s": round(T / (ms / 1e3), 1), "expert_GB": round(nbytes / 1e9, 3),
            "expert_GB_s": round(nbytes / (ms / 1e3) / 1e9, 1), "status": int(status)}


def _lib_err():
    from integer_inference_engine_amd import _lib
    return _lib.last_error()


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--replicas", type=int, default=384)
    ap.add_argument("--cpu-seconds", type=float, default=2.0, help="seconds per CPU-baseline repetition")
    ap.add_argument("--cpu-reps", type=int, default=5, help="CPU-baseline repetitions (median reported)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--decode-tokens", type=int, default=32, help="8B-shape b=1 decode leg (0 = skip)")
    ap.add_argument("--prefill-tokens", type=int, default=2048, help="config-3 layer prefill leg (0 = skip)")
    ap.add_argument("--c5-tokens", type=int, default=64, help="config-5 ragged batch decode leg (0 = skip)")
    ap.add_argument("--moe-tokens", type=int, default=64, help="config-4 MoE block leg (0 = skip)")
    ap.add_argument("--cpu-worker", default=None, help=argparse.SUPPRESS)
    ap.add_argument("--cpu-port", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device-to-device copy 3 times (HBM counter calibration)")
    args = ap.parse_args()
    if args.cpu_worker:
        cpu_worker(args.cpu_worker, args.cpu_seconds, args.cpu_reps, args.cpu_port)
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build measures ONE MI355X; --gpus {args.gpus} is not supported "
              "(one GPU's share of a sharded model is what runs here; the sharding itself is not built)",
              file=sys.stderr)
        return 2

    import ctypes
    import torch
    from integer_inference_engine_amd import _lib
    if args.copy_calibration:
        src = torch.ones(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": 1 << 30, "launches": 3}))
        return 0
    so = _lib.lib()
    assert _lib.device_available(), "no usable gfx950 device"
    R = args.replicas
    N = K * R
    rng = np.random.default_rng(2026)
    print(f"[bench] generating {R} replicas of a {K}x{K} Q1_0 weight", file=sys.stderr, flush=True)
    bits = rng.integers(0, 256, size=(N, NB, 16), dtype=np.uint8)
    scale = codec_scales(rng, (N, NB))
    h = so.bonsai_q1_register_weight(bits.ctypes.data, scale.ctypes.data, N, NB)
    assert h >= 0, _lib.last_error()
    nn, nbb, sb = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    so.imie_q1_weight_info(h, ctypes.byref(nn), ctypes.byref(nbb), ctypes.byref(sb))
    scale_bytes = int(sb.value)
    x_host = rng.integers(-127, 128, size=(1, K), dtype=np.int64)
    x = torch.from_numpy(x_host).cuda()
    out = torch.empty((1, N), dtype=torch.int64, device="cuda")
    stream = torch.cuda.Stream()          # a real (non-null) stream shared by the kernels and the timing events
    torch.cuda.set_stream(stream)
    sp = ctypes.c_void_p(stream.cuda_stream)

    def step():
        rc = so.imie_q1_apply_dev(h, ctypes.c_void_p(x.data_ptr()), 1, 16, ctypes.c_void_p(out.data_ptr()), sp)
        assert rc == 0, _lib.last_error()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # exactness spot check of replica 0 against the library's independent thread-per-output kernel
    b0 = torch.from_numpy(np.ascontiguousarray(bits[:K])).cuda()
    s0 = torch.from_numpy(np.ascontiguousarray(scale[:K])).cuda()
    chk = torch.empty((1, K), dtype=torch.int64, device="cuda")
    assert so.imie_q1_linear_simple_dev(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(b0.data_ptr()),
                                        ctypes.c_void_p(s0.data_ptr()), 1, K, NB, 16, ctypes.c_void_p(chk.data_ptr()),
                                        sp) == 0
    torch.cuda.synchronize()
    exact = bool(torch.equal(chk[0], out[0, :K]))

    # timed region: the K steps alone (no profiler events on the stream)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for _ in range(args.steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1)
    # the dominant kernel's launch duration: the same K steps again with HIP events around each launch, on the
    # stream the kernel runs on
    so.imie_profile_begin()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    kms, kcnt = ctypes.c_double(), ctypes.c_int64()
    so.imie_profile_read(1, ctypes.byref(kms), ctypes.byref(kcnt))
    pms, pcnt = ctypes.c_double(), ctypes.c_int64()
    so.imie_profile_read(0, ctypes.byref(pms), ctypes.byref(pcnt))
    so.imie_profile_end()

    step_bytes = R * matvec_bytes(scale_bytes)
    value = step_bytes * args.steps / (ms / 1e3) / 1e9
    # per-launch event pairs add their own marker and cache-release time to each launch; when every step is
    # exactly one launch of the dominant kernel (no prep kernel), the timed region's events on the same stream
    # bracket back-to-back launches of that kernel alone, and their mean is the launch duration
    k_avg_iso_s = kms.value / max(1, kcnt.value) / 1e3
    k_avg_s = ms / args.steps / 1e3 if (kcnt.value == args.steps and pcnt.value == 0) else k_avg_iso_s
    achieved = step_bytes / k_avg_s / 1e9
    traffic = None
    tf = ROOT / "profiles" / "q1_matvec_c1_traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("traffic_bytes_per_launch")

    # byte-exactness of the timed launch: every replica's 4096 outputs against the CPU Q1 linear (the reference C
    # kernel when built) on the same weights and x
    out_host = out.cpu().numpy()
    ref_fn, ref_kind = _ref_q1()
    ref_out = np.empty((1, K), dtype=np.int64)
    bad = 0
    for r in range(R):
        br = np.ascontiguousarray(bits[r * K:(r + 1) * K])
        sr = np.ascontiguousarray(scale[r * K:(r + 1) * K])
        assert ref_fn(x_host.ctypes.data, br.ctypes.data, sr.ctypes.data, 1, K, NB, 16, ref_out.ctypes.data) == 0
        bad += int(not np.array_equal(ref_out[0], out_host[0, r * K:(r + 1) * K]))

    cpu = None
    if not args.no_cpu_baseline:
        # the host's CPU share on the GPU box (OMP_NUM_THREADS there, else the cores this process may use), and one
        # thread; each the median of --cpu-reps repetitions of --cpu-seconds
        share = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
        res = {}
        with tempfile.TemporaryDirectory() as td:
            npz = os.path.join(td, "c1.npz")
            np.savez(npz, x=x_host, bits=bits[:K], scale=scale[:K], out=out_host[:, :K])
            # the reference C kernel at the job's share and at one thread, then the repo's own C restatement
            # (oracle/c) at the share: the restatement is the baseline that does not need the reference tree
            for key, threads, impl in (("ref", share, []), ("ref1", 1, []), ("port", share, ["--cpu-port"])):
                env = dict(os.environ, OMP_NUM_THREADS=str(threads), OMP_PROC_BIND="close")
                r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--cpu-worker", npz, "--cpu-seconds",
                                    str(args.cpu_seconds), "--cpu-reps", str(args.cpu_reps), *impl], env=env,
                                   capture_output=True, text=True, timeout=600)
                if r.returncode != 0:
                    print(r.stderr[-2000:], file=sys.stderr)
                    break
                res[key] = json.loads(r.stdout.strip().splitlines()[-1])
        if "ref" in res and "ref1" in res:
            c, c1 = res["ref"], res["ref1"]
            cp = res.get("port")
            cpu = {"value": round(c["value"], 3), "unit": "GB/s", "cores": share, "kind": c["kind"],
                   "single_thread_value": round(c1["value"], 3),
                   "port_value": round(cp["value"], 3) if cp else None, "cpu_model": cpu_model(),
                   "host_cpus": os.cpu_count(),
                   "sample": f"config-1 4096x4096 Q1_0 matvec (int64 codec-range scales), median of "
                             f"{args.cpu_reps} x {args.cpu_seconds:.0f} s runs at {share} threads "
                             f"({c['calls']} calls) and at 1 thread ({c1['calls']} calls); port_value: the repo's C "
                             f"restatement (oracle/c) at {share} threads; output byte-equal to GPU: "
                             f"{c['match'] and c1['match'] and (cp is None or cp['match'])}"}

    dec = None
    # the device's practical read ceiling (streaming nontemporal loads over a buffer of the same size), to set the
    # matvec's fraction of the published peak beside what the memory system actually sustains
    rpk = ctypes.c_double()
    read_peak = rpk.value / 1e9 if so.imie_hbm_read_peak(step_bytes, ctypes.byref(rpk)) == 0 else None

    if args.decode_tokens > 0 or args.c5_tokens > 0:
        del bits, scale
        so.bonsai_q1_free_weights()
        print("[bench] 8B-shape decode leg", file=sys.stderr, flush=True)
        dec = decode_leg(so, torch, args.decode_tokens, c5_tokens=args.c5_tokens)

    pre = None
    if args.prefill_tokens > 0:
        print("[bench] config-3 prefill leg", file=sys.stderr, flush=True)
        pre = prefill_leg(so, torch, args.prefill_tokens)

    moe = None
    if args.moe_tokens > 0:
        print("[bench] config-4 MoE leg", file=sys.stderr, flush=True)
        moe = moe_leg(so, torch, T=args.moe_tokens)

    line = {
        "metric": "Q1 matvec HBM GB/s (% of peak); 8B-shape decode tok/s b=1; byte-exact",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int64 (int8 MFMA limbs, i32 accumulate)", "data": "synthetic",
        "config": {"workload": f"config-1 Q1_0 matvec 4096x4096, b=1, rotated over {R} resident replicas "
                               f"(one launch = {R} matvecs, {step_bytes / 1e9:.2f} GB)",
                   "replicas": R, "scale_bytes": scale_bytes, "frac": 16, "byte_exact_replica0": exact,
                   "byte_exact_all_replicas": bad == 0, "replicas_checked": R, "checked_against": ref_kind,
                   "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
                   "us_per_matvec": round(ms / args.steps / R * 1e3, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": "profiles/q1_matvec_c1_traffic.json: rocprofv3 --pmc FETCH_SIZE and "
                                       "WRITE_SIZE of this launch, copy-calibrated" if traffic else None,
                     "frac_step": round(value / HBM_PEAK_GBS, 4),
                     "kernel": "q1_gemv_mfma_kernel", "kernel_avg_us": round(k_avg_s * 1e6, 3),
                     "kernel_avg_us_event_pairs": round(k_avg_iso_s * 1e6, 3),
                     "measured_read_peak": round(read_peak, 1) if read_peak else None,
                     "frac_of_measured_read_peak": round(achieved / read_peak, 4) if read_peak else None,
                     "prep_avg_us": round(pms.value / max(1, pcnt.value) * 1e3, 3)},
        "cpu_baseline": cpu,
        "decode_8b_b1": {k: v for k, v in dec.items() if k != "_c5"} if dec and args.decode_tokens > 0 else None,
        "decode_c5_batch32": dec.get("_c5") if dec else None,
        "prefill_8b_layer": pre,
        "moe_c4": moe,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
