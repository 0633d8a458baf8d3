"""Bonsai hot-path kernels and the resident forward on gfx950 vs the oracle, byte for byte.

Parity gates after bonsai/tests/test_bonsai_gpu.py:174-343 and test_bonsai_smoke.py:358-432, 1231-1632."""
import numpy as np
import pytest

from oracle import attention as oatt, bonsai_model as obm, fixedpoint as fx, prng, workloads
from oracle.q1 import q1_rows
from oracle.rope import build_rope_tables
from tests.bonsai_gpu_harness import register_model

pytestmark = pytest.mark.gpu
I64_MIN, I64_MAX = -(1 << 63), (1 << 63) - 1


def assert_same(got, want, what=""):
    assert got is not None, f"{what}: producer declined"
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    bad = np.flatnonzero(np.asarray(got).ravel() != np.asarray(want).ravel())
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[0]}: {got.ravel()[bad[0]]} != {want.ravel()[bad[0]]}"


@pytest.mark.parametrize("rows,cols,mag", [(1, 4096, 25), (40, 128, 14), (7, 4096, 40), (3, 96, 57), (2, 12288, 20),
                                           (70, 4096, 30), (64, 2560, 20)])
def test_rmsnorm_matches_oracle(gpu, rows, cols, mag):
    x = prng.uniform_int(mag, 1, (rows, cols), -(1 << mag), 1 << mag)
    g = prng.uniform_int(mag, 2, (cols,), 1 << 15, 1 << 17)
    assert_same(gpu.rmsnorm_gpu(x, 16, 1, None), fx.rmsnorm(x, 16, 1, None), "no gain")
    if mag <= 40:
        assert_same(gpu.rmsnorm_gpu(x, 16, 1, g), fx.rmsnorm(x, 16, 1, g), "gain")


def test_rmsnorm_beyond_128_bit_ssq_is_refused(gpu):
    # 96 values near 2^62: ssq ~ 2^130.6 -> the producer returns rc 4 (bonsai_q1_kernel.c:262-268 rule);
    # the big-int oracle still computes it.
    x = prng.uniform_int(62, 1, (3, 96), -(1 << 62), 1 << 62)
    assert gpu.rmsnorm_gpu(x, 16, 1, None) is None
    assert fx.rmsnorm(x, 16, 1, None).shape == (3, 96)


def test_rmsnorm_refuses_where_oracle_raises(gpu):
    # bonsai/tests/test_bonsai_gpu.py:194-207 lockstep: gain envelope -> rc 4 (None) where the oracle raises
    x = np.array([[1 << 20, -(1 << 20), 3, 4]], dtype=np.int64)
    g = np.array([1 << 60, 1, 1, 1], dtype=np.int64)
    with pytest.raises(OverflowError):
        fx.rmsnorm(x, 16, 1, g)
    assert gpu.rmsnorm_gpu(x, 16, 1, g) is None
    # ssq beyond 128 bits: refused by the producer, computed by the big-int oracle
    big = np.full((1, 8), I64_MIN, dtype=np.int64)
    assert gpu.rmsnorm_gpu(big, 16, 1, None) is None


def _fused_rmsnorm(x, frac, eps, g):
    import ctypes
    from integer_inference_engine_amd import _lib
    x = np.ascontiguousarray(x, dtype=np.int64)
    out = np.empty_like(x)
    gg = None if g is None else np.ascontiguousarray(g, dtype=np.int64)
    rc = _lib.lib().imie_rmsnorm_fused_gpu(x.ctypes.data, x.shape[0], x.shape[1], frac, eps,
                                           None if gg is None else gg.ctypes.data, out.ctypes.data)
    return None if rc != 0 else out


@pytest.mark.parametrize("rows,cols,mag", [(1, 4096, 25), (7, 4096, 40), (3, 2560, 30), (2, 128, 50), (1, 640, 61)])
def test_fused_rmsnorm_prep_matches_oracle(gpu, rows, cols, mag):
    # the decode's RMSNorm + digit-table producer: per-row extremes decide max|n| (all-negative and
    # all-positive rows included)
    x = prng.uniform_int(mag, 3, (rows, cols), -(1 << mag), 1 << mag)
    x[0] = np.abs(x[0])
    if rows > 1:
        x[1] = -np.abs(x[1]) - 1
    g = prng.uniform_int(mag, 4, (cols,), -(1 << 17), 1 << 17)
    ssq_over = any(sum(int(v) * int(v) for v in row) >= 1 << 128 for row in x)   # producer refuses (rc 4)
    for gain in (g, None):
        try:
            want = None if ssq_over else fx.rmsnorm(x, 16, 1, gain)
        except OverflowError:
            want = None
        got = _fused_rmsnorm(x, 16, 1, gain)
        if want is None:
            assert got is None
        else:
            assert_same(got, want, f"fused gain={gain is not None}")


def test_fused_rmsnorm_refusals(gpu):
    # gain envelope decided by the negative extreme alone; ssq beyond 128 bits; one huge element
    x = np.zeros((1, 128), dtype=np.int64)
    x[0, :4] = [3, -(1 << 20), 5, 7]
    g = np.ones(128, dtype=np.int64)
    g[5] = 1 << 50
    with pytest.raises(OverflowError):
        fx.rmsnorm(x, 16, 1, g)
    assert _fused_rmsnorm(x, 16, 1, g) is None
    g[5] = 1 << 20
    assert_same(_fused_rmsnorm(x, 16, 1, g), fx.rmsnorm(x, 16, 1, g), "just inside the envelope")
    big = np.full((1, 128), I64_MIN, dtype=np.int64)
    assert _fused_rmsnorm(big, 16, 1, g) is None
    assert _fused_rmsnorm(big, 16, 1, None) is None


def test_silu_matches_oracle_including_int64_extremes(gpu):
    x = np.concatenate([prng.uniform_int(3, 1, (5000,), -(1 << 40), 1 << 40),
                        [I64_MIN, I64_MAX, I64_MIN + 1, 0, 1, -1, 1 << 62, -(1 << 62)]]).astype(np.int64)
    for frac in (16, 29):
        assert np.array_equal(gpu.silu_gpu(x, frac), fx.silu_wrap(x, frac) if frac == 16 else
                              (x * fx.sigmoid(x, frac)) >> np.int64(frac))


def test_rope_matches_oracle_and_guards(gpu):
    cos, sin = build_rope_tables(64, 32, 1_000_000, 16)
    x = prng.uniform_int(4, 1, (10, 4, 32), -(1 << 22), 1 << 22)
    pos = np.arange(10) * 3 + 5
    from oracle.rope import apply_neox_rows
    assert np.array_equal(gpu.rope_neox_gpu(x, pos, cos, sin, 16), apply_neox_rows(x, cos[pos], sin[pos], 16))
    huge = np.full((1, 1, 32), 1 << 50, dtype=np.int64)
    assert gpu.rope_neox_gpu(huge, [1], cos, sin, 16) is None


def test_argmax_lowest_index_on_ties(gpu):
    z = prng.uniform_int(5, 1, (6, 3001), -(1 << 40), 1 << 40)
    z[1, :] = 7                      # all ties -> index 0
    z[2, 2999] = z[2, 5] = I64_MAX   # first max wins
    assert list(gpu.argmax_gpu(z)) == list(np.argmax(z, axis=1))


@pytest.mark.parametrize("H,Hkv,hd,M,start", [(32, 8, 128, 9, 0), (4, 2, 32, 33, 17), (8, 8, 64, 1, 300)])
def test_attention_prefill_matches_oracle(gpu, H, Hkv, hd, M, start):
    L = start + M
    q = prng.uniform_int(H, 1, (H, M, hd), -(1 << 20), 1 << 20)
    k, v = workloads.kv_fill(H, 2, Hkv, L, hd)
    got = gpu.attention_prefill_gpu(q, k, v, start, 16, fx.inv_sqrt_fp(hd, 16))
    assert got is not None
    assert_same(got, oatt.attention_cached(q, k, v, start, 16, fx.inv_sqrt_fp(hd, 16)), "prefill attention")


def test_attention_fail_loud_like_reference(gpu):
    # bonsai/tests/test_bonsai_smoke.py:1600-1632 shapes: q,k at 2^40 with hd 8 overflow the QK bound
    q = np.full((2, 1, 8), 1 << 40, dtype=np.int64)
    k = np.full((1, 1, 8), 1 << 40, dtype=np.int64)
    v = np.ones((1, 1, 8), dtype=np.int64)
    with pytest.raises(OverflowError):
        oatt.attention_cached(q, k, v, 0, 16, 5793)
    assert gpu.attention_prefill_gpu(q, k, v, 0, 16, 5793) is None


def test_attention_decode_batched_ragged(gpu):
    B, H, Hkv, hd, cap = 5, 8, 2, 64, 300
    lengths = [1, 17, 64, 65, 300]
    q = prng.uniform_int(9, 1, (B, H, hd), -(1 << 20), 1 << 20)
    K = prng.uniform_int(9, 2, (B, Hkv, cap, hd), -(1 << 20), 1 << 20)
    V = prng.uniform_int(9, 3, (B, Hkv, cap, hd), -(1 << 20), 1 << 20)
    got = gpu.attention_decode_batched_gpu(q, K, V, lengths, 16, fx.inv_sqrt_fp(hd, 16))
    want = oatt.attention_decode_batched(q, [K[b, :, :lengths[b]] for b in range(B)],
                                         [V[b, :, :lengths[b]] for b in range(B)], 16, fx.inv_sqrt_fp(hd, 16))
    assert_same(got, want, "decode attention")


def _oracle_prefill(model, ids):
    cfg = model["cfg"]
    c = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    x = q1_rows(*model["embed"], ids)
    ks, vs = [], []
    for layer in model["layers"]:
        x, kn, vn = obm.layer_forward(x, layer, c, model["cos"], model["sin"], 16, None, None, 0)
        ks.append(kn); vs.append(vn)
    return x, np.stack(ks), np.stack(vs)


@pytest.mark.parametrize("T", [1, 4, 17, 32])
def test_prefill_monolith_logits_and_kv_export(gpu, T):
    model = workloads.small_bonsai(seed=T)
    cfg = model["cfg"]
    w, g = register_model(gpu, model)
    ids = prng.uniform_int(T, 99, (T,), 0, cfg["vocab"])
    x0 = q1_rows(*model["embed"], ids)
    dims = (T, cfg["d"], cfg["n_layers"], cfg["H"], cfg["Hkv"], cfg["hd"], cfg["dff"])
    logits, k, v = gpu.prefill_forward_gpu(x0, dims, w, g, 16, 1, fx.inv_sqrt_fp(cfg["hd"], 16), export_kv=True)
    x, ks, vs = _oracle_prefill(model, ids)
    want = obm.head_logits(model, x[-1:], 16)[0]
    assert_same(logits, want, "logits")
    assert_same(k, ks, "K export")
    assert_same(v, vs, "V export")


def test_decode_ctx_greedy_generation_matches_oracle(gpu):
    model = workloads.small_bonsai(seed=42)
    cfg = model["cfg"]
    w, g = register_model(gpu, model)
    B, T0, steps = 3, [5, 9, 2], 6
    prompts = [prng.uniform_int(42, 200 + b, (T0[b],), 0, cfg["vocab"]) for b in range(B)]
    c = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    ctx = gpu.decode_ctx_create((B, cfg["n_layers"], cfg["H"], cfg["Hkv"], cfg["hd"], cfg["d"], cfg["dff"],
                                 cfg["vocab"]), w, g, 16, 1, fx.inv_sqrt_fp(cfg["hd"], 16), 64)
    assert ctx is not None
    caches, nxt = [], []
    for b in range(B):
        x, ks, vs = _oracle_prefill(model, prompts[b])
        assert gpu.decode_ctx_seed_seq(ctx, b, ks, vs)
        caches.append(([ks[li] for li in range(len(ks))], [vs[li] for li in range(len(vs))]))
        nxt.append(int(np.argmax(obm.head_logits(model, x[-1:], 16)[0])))
    pos = list(T0)
    for _ in range(steps):
        x_in = q1_rows(*model["embed"], nxt)
        logits = gpu.decode_step(ctx, x_in, pos, cfg["vocab"])
        assert logits is not None
        for b in range(B):
            xb = x_in[b:b + 1]
            kc, vc = caches[b]
            for li, layer in enumerate(model["layers"]):
                xb, kn, vn = obm.layer_forward(xb, layer, c, model["cos"], model["sin"], 16, kc[li], vc[li], pos[b])
                kc[li] = np.concatenate([kc[li], kn], axis=1)
                vc[li] = np.concatenate([vc[li], vn], axis=1)
            want = obm.head_logits(model, xb, 16)[0]
            assert_same(logits[b], want, f"seq {b} pos {pos[b]}")
        nxt = [int(v) for v in np.argmax(logits, axis=1)]
        pos = [p + 1 for p in pos]
    gpu.decode_ctx_free(ctx)


@pytest.mark.parametrize("graph", [0, 1])
def test_device_greedy_decode_matches_oracle(gpu, graph):
    """imie_net_decode_dev: embed -> layers -> head -> argmax on the device for B=3 ragged sequences; the graph
    variant replays one captured step, so steps 2.. exercise the replay (positions advance on the device)."""
    import ctypes
    import torch
    from integer_inference_engine_amd import _lib
    model = workloads.small_bonsai(seed=43)
    cfg = model["cfg"]
    w, g = register_model(gpu, model)
    B, T0, steps = 3, [5, 9, 2], 7
    prompts = [prng.uniform_int(43, 300 + b, (T0[b],), 0, cfg["vocab"]) for b in range(B)]
    c = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    ctx = gpu.decode_ctx_create((B, cfg["n_layers"], cfg["H"], cfg["Hkv"], cfg["hd"], cfg["d"], cfg["dff"],
                                 cfg["vocab"]), w, g, 16, 1, fx.inv_sqrt_fp(cfg["hd"], 16), 64)
    assert ctx is not None
    caches, first = [], []
    for b in range(B):
        x, ks, vs = _oracle_prefill(model, prompts[b])
        assert gpu.decode_ctx_seed_seq(ctx, b, ks, vs)
        caches.append(([ks[li] for li in range(len(ks))], [vs[li] for li in range(len(vs))]))
        first.append(int(np.argmax(obm.head_logits(model, x[-1:], 16)[0])))
    # oracle greedy continuation
    want_tok, nxt, pos = [], list(first), list(T0)
    for _ in range(steps):
        x_in = q1_rows(*model["embed"], nxt)
        logits = []
        for b in range(B):
            xb = x_in[b:b + 1]
            kc, vc = caches[b]
            for li, layer in enumerate(model["layers"]):
                xb, kn, vn = obm.layer_forward(xb, layer, c, model["cos"], model["sin"], 16, kc[li], vc[li], pos[b])
                kc[li] = np.concatenate([kc[li], kn], axis=1)
                vc[li] = np.concatenate([vc[li], vn], axis=1)
            logits.append(obm.head_logits(model, xb, 16)[0])
        nxt = [int(np.argmax(lg)) for lg in logits]
        want_tok.append(nxt)
        pos = [p + 1 for p in pos]
    so = _lib.lib()
    eb = torch.from_numpy(np.ascontiguousarray(model["embed"][0])).cuda()
    es = torch.from_numpy(np.ascontiguousarray(model["embed"][1])).cuda()
    ids = torch.tensor(first, dtype=torch.int64, device="cuda")
    lg = torch.empty((B, cfg["vocab"]), dtype=torch.int64, device="cuda")
    hist = torch.full((steps, B), -1, dtype=torch.int64, device="cuda")
    s = torch.cuda.Stream()
    sp = ctypes.c_void_p(s.cuda_stream)
    so.imie_net_status(ctx, 1, sp)
    rc = so.imie_net_decode_dev(ctx, ctypes.c_void_p(eb.data_ptr()), ctypes.c_void_p(es.data_ptr()),
                                ctypes.c_void_p(ids.data_ptr()), ctypes.c_void_p(lg.data_ptr()),
                                ctypes.c_void_p(hist.data_ptr()), steps, graph, sp)
    assert rc == 0, _lib.last_error()
    assert so.imie_net_status(ctx, 0, sp) == 0
    s.synchronize()
    assert hist.cpu().numpy().tolist() == want_tok
    assert_same(lg.cpu().numpy(), np.stack(logits), "last-step logits")
    for b in range(B):
        for li in range(cfg["n_layers"]):
            k = np.empty((cfg["Hkv"], T0[b] + steps, cfg["hd"]), dtype=np.int64)
            v = np.empty_like(k)
            assert so.imie_net_export_kv(ctx, li, b, T0[b] + steps, k.ctypes.data, v.ctypes.data) == 0
            assert np.array_equal(k, caches[b][0][li][:, :T0[b] + steps]) and np.array_equal(v, caches[b][1][li][:, :T0[b] + steps])
    gpu.decode_ctx_free(ctx)


@pytest.mark.parametrize("graph", [0, 1])
def test_device_sampled_decode_matches_oracle(gpu, graph):
    """imie_net_decode_sampled_dev: each token equals the oracle's sample_token(logits, cfg, len(ids), 16, ids) over
    the oracle model's logits (top-p with top-k, temperature, repetition penalty and a 2-gram ban)."""
    import ctypes
    from types import SimpleNamespace
    import torch
    from integer_inference_engine_amd import _lib
    from integer_inference_engine_amd.sampler_gpu import config_c
    from oracle import sampler as osm
    model = workloads.small_bonsai(seed=44)
    cfg = model["cfg"]
    w, g = register_model(gpu, model)
    B, T0, steps, hld = 3, [5, 9, 2], 6, 32
    scfg = SimpleNamespace(mode="top_p", temperature=0.5, top_k=12, top_p=0.9, min_p=0.0, seed=11,
                           rep_penalty=13107, no_repeat_ngram=2)
    c = config_c(scfg, 16)
    draw = lambda row, ids: osm.sample_token(row, "top_p", 16, inv_temp=c.inv_temp, top_k=c.top_k, top_p_fp=c.top_p,
                                             seed=scfg.seed, position=len(ids), hist=ids, rep_penalty=c.rep_penalty,
                                             no_repeat_ngram=c.no_repeat_ngram)
    prompts = [prng.uniform_int(44, 400 + b, (T0[b],), 0, cfg["vocab"]) for b in range(B)]
    lc = {"H": cfg["H"], "Hkv": cfg["Hkv"], "hd": cfg["hd"]}
    ctx = gpu.decode_ctx_create((B, cfg["n_layers"], cfg["H"], cfg["Hkv"], cfg["hd"], cfg["d"], cfg["dff"],
                                 cfg["vocab"]), w, g, 16, 1, fx.inv_sqrt_fp(cfg["hd"], 16), 64)
    assert ctx is not None
    caches, ids = [], []
    for b in range(B):
        x, ks, vs = _oracle_prefill(model, prompts[b])
        assert gpu.decode_ctx_seed_seq(ctx, b, ks, vs)
        caches.append(([ks[li] for li in range(len(ks))], [vs[li] for li in range(len(vs))]))
        toks = [int(t) for t in prompts[b]]
        toks.append(draw(obm.head_logits(model, x[-1:], 16)[0], toks))
        ids.append(toks)
    first = [t[-1] for t in ids]
    hist0 = np.full((B, hld), -1, dtype=np.int64)
    for b in range(B):
        hist0[b, :len(ids[b])] = ids[b]
    len0 = [len(t) for t in ids]
    pos = list(T0)
    for _ in range(steps):
        x_in = q1_rows(*model["embed"], [t[-1] for t in ids])
        for b in range(B):
            xb = x_in[b:b + 1]
            kc, vc = caches[b]
            for li, layer in enumerate(model["layers"]):
                xb, kn, vn = obm.layer_forward(xb, layer, lc, model["cos"], model["sin"], 16, kc[li], vc[li], pos[b])
                kc[li] = np.concatenate([kc[li], kn], axis=1)
                vc[li] = np.concatenate([vc[li], vn], axis=1)
            ids[b].append(draw(obm.head_logits(model, xb, 16)[0], ids[b]))
        pos = [p + 1 for p in pos]
    so = _lib.lib()
    eb = torch.from_numpy(np.ascontiguousarray(model["embed"][0])).cuda()
    es = torch.from_numpy(np.ascontiguousarray(model["embed"][1])).cuda()
    dids = torch.tensor(first, dtype=torch.int64, device="cuda")
    lg = torch.empty((B, cfg["vocab"]), dtype=torch.int64, device="cuda")
    hist = torch.from_numpy(hist0).cuda()
    hlen = torch.tensor(len0, dtype=torch.int64, device="cuda")
    s = torch.cuda.Stream()
    sp = ctypes.c_void_p(s.cuda_stream)
    so.imie_net_status(ctx, 1, sp)
    rc = so.imie_net_decode_sampled_dev(ctx, ctypes.c_void_p(eb.data_ptr()), ctypes.c_void_p(es.data_ptr()),
                                        ctypes.c_void_p(dids.data_ptr()), ctypes.c_void_p(lg.data_ptr()),
                                        ctypes.byref(c), ctypes.c_void_p(hist.data_ptr()), hld,
                                        ctypes.c_void_p(hlen.data_ptr()), steps, graph, sp)
    assert rc == 0, _lib.last_error()
    assert so.imie_net_status(ctx, 0, sp) == 0
    s.synchronize()
    got = hist.cpu().numpy()
    assert hlen.cpu().numpy().tolist() == [len(t) for t in ids]
    for b in range(B):
        assert got[b, :len(ids[b])].tolist() == ids[b], b
    gpu.decode_ctx_free(ctx)
