"""north-mini-code resident preprocessing and attention bank vs the oracle (the reference's resident layer rung,
north-mini-code tests of qk_cuda.ResidentAttentionCache / rmsnorm_router): byte-exact outputs, routes, gates and
K/V lengths; guards and unbound experts fail closed."""
import numpy as np
import pytest

from oracle import fixedpoint as fx
from oracle import nmc_block as onb
from oracle import qk
from oracle.rope import build_rope_tables

pytestmark = pytest.mark.gpu
FA, FW = 16, 24
D, H, HKV, HD, E, USED, EFF = 256, 4, 2, 64, 8, 2, 256
CAP = 40


def _weights(seed):
    from integer_inference_engine_amd import qk_gpu
    rng = np.random.default_rng(seed)
    W, handles, experts, ehandles = {}, {}, {}, {}
    for i, (name, of, nb, qt) in enumerate((("wq", H * HD, D // 256, 0), ("wk", HKV * HD, D // 256, 1),
                                            ("wv", HKV * HD, D // 256, 0), ("wo", D, H * HD // 256, 1))):
        raw = qk.random_blocks(seed, i, of, nb, qt)
        W[name] = qk.dequant(raw, of, nb, qt, FW)
        handles[name] = qk_gpu.register_weight(raw, of, nb, qt)
    W["gain"] = rng.integers(1 << 15, (1 << 17) + 1, size=D, dtype=np.int64)
    W["router"] = rng.integers(-(1 << 20), 1 << 20, size=(E, D), dtype=np.int64)
    handles["gain"] = qk_gpu.register_i64(W["gain"].reshape(1, D))
    handles["router"] = qk_gpu.register_i64(W["router"])
    for e in range(E):
        g = qk.random_blocks(seed + 1, 10 + 3 * e, EFF, D // 256, 0)
        u = qk.random_blocks(seed + 1, 11 + 3 * e, EFF, D // 256, 0)
        dn = qk.random_blocks(seed + 1, 12 + 3 * e, D, EFF // 256, 1)
        experts[e] = {"gate": qk.dequant(g, EFF, D // 256, 0, FW), "up": qk.dequant(u, EFF, D // 256, 0, FW),
                      "down": qk.dequant(dn, D, EFF // 256, 1, FW)}
        ehandles[e] = (qk_gpu.register_weight(g, EFF, D // 256, 0), qk_gpu.register_weight(u, EFF, D // 256, 0),
                       qk_gpu.register_weight(dn, D, EFF // 256, 1))
    return W, handles, experts, ehandles


CFG = {"fa": FA, "fw": FW, "H": H, "Hkv": HKV, "hd": HD, "used": USED, "eps": 1}


def test_rmsnorm_router_matches_oracle(gpu):
    from integer_inference_engine_amd import qk_gpu
    W, hs, _, _ = _weights(3)
    rng = np.random.default_rng(4)
    x = rng.integers(-(1 << 20), 1 << 20, size=(3, D), dtype=np.int64)
    got = qk_gpu.rmsnorm_router(hs["gain"], hs["router"], x, USED, FA, FW, 1)
    assert got is not None
    h = fx.rmsnorm(x, FA, 1, W["gain"])
    logits = onb.router_logits(h, W["router"], FW)
    sel, gates = qk.moe_route(logits, USED, FA)
    assert np.array_equal(got[0], h)
    assert np.array_equal(got[1], sel.astype(np.int32))
    assert np.array_equal(got[2], gates)
    # a router row whose unshifted sum leaves int64: the producer refuses (None), the oracle raises
    big = np.full((1, D), (1 << 40), dtype=np.int64)
    hb = qk_gpu.register_i64(np.full((1, D), 1 << 20, dtype=np.int64))
    rb = qk_gpu.register_i64(np.full((E, D), 1 << 40, dtype=np.int64))
    assert qk_gpu.rmsnorm_router(hb, rb, big, USED, FA, FW, 1) is None
    qk_gpu.free_all()


@pytest.mark.parametrize("window,rope", [(None, False), (6, True), (3, True), (None, True)])
def test_bank_apply_matches_oracle(gpu, window, rope):
    from integer_inference_engine_amd import qk_gpu
    W, hs, _, _ = _weights(5)
    cos, sin = build_rope_tables(CAP, HD, base=50000, frac=FA)
    bank = qk_gpu.ResidentAttentionCache(1, CAP, D, H, HKV, HD, FA, cos, sin)
    rng = np.random.default_rng(6)
    L0 = 7
    kc = np.zeros((HKV, CAP, HD), dtype=np.int64)
    vc = np.zeros_like(kc)
    kc[:, :L0] = rng.integers(-(1 << 17), 1 << 17, size=(HKV, L0, HD))
    vc[:, :L0] = rng.integers(-(1 << 17), 1 << 17, size=(HKV, L0, HD))
    bank.import_layer(0, kc[:, :L0], vc[:, :L0])
    inv = fx.inv_sqrt_fp(HD, FA)
    for step in range(4):
        pos = L0 + step
        hrow = rng.integers(-(1 << 18), 1 << 18, size=(1, D), dtype=np.int64)
        got = bank.apply(0, hs["wq"], hs["wk"], hs["wv"], hs["wo"], hrow, FW, window, rope)
        q = qk.linear(hrow, W["wq"], FW).reshape(H, HD)
        k = qk.linear(hrow, W["wk"], FW).reshape(HKV, HD)
        v = qk.linear(hrow, W["wv"], FW).reshape(HKV, HD)
        if rope:
            from oracle.rope import apply_interleaved
            q = apply_interleaved(q[:, None, :], cos[pos:pos + 1], sin[pos:pos + 1], FA)[:, 0, :]
            k = apply_interleaved(k[:, None, :], cos[pos:pos + 1], sin[pos:pos + 1], FA)[:, 0, :]
        kc[:, pos], vc[:, pos] = k, v
        att = onb.attention_step(q, kc, vc, pos, window, FA, inv).reshape(1, H * HD)
        assert np.array_equal(got, qk.linear(att, W["wo"], FW)), (window, rope, step)
        assert bank.length(0) == pos + 1
    assert bank.workspace_bytes() > 2 * HKV * CAP * HD * 8
    bank.close()
    qk_gpu.free_all()


def test_bank_moe_chain_matches_oracle(gpu):
    """Two consecutive MoE layers: begin (host x) -> bind the reported cold experts -> continue retained ->
    begin (retained) -> continue published, against two oracle block steps; experts bound lazily."""
    from integer_inference_engine_amd import qk_gpu
    W, hs, experts, eh = _weights(7)
    cos, sin = build_rope_tables(CAP, HD, base=50000, frac=FA)
    bank = qk_gpu.ResidentAttentionCache(2, CAP, D, H, HKV, HD, FA, cos, sin)
    rng = np.random.default_rng(8)
    caches = []
    for layer in range(2):
        L0 = 5 + 2 * layer
        kc = np.zeros((HKV, CAP, HD), dtype=np.int64)
        vc = np.zeros_like(kc)
        kc[:, :L0] = rng.integers(-(1 << 17), 1 << 17, size=(HKV, L0, HD))
        vc[:, :L0] = rng.integers(-(1 << 17), 1 << 17, size=(HKV, L0, HD))
        bank.import_layer(layer, kc[:, :L0], vc[:, :L0])
        bank.configure_moe_layer(layer, E, USED, D, EFF)
        caches.append([kc, vc, L0])
    bank.bind_moe_expert(1, 0, *eh[0])                  # one expert of layer 1 bound up front
    x = rng.integers(-(1 << 20), 1 << 20, size=(1, D), dtype=np.int64)
    specs = [(None, False), (4, True)]
    state, want = x, x
    for layer in range(2):
        window, rope = specs[layer]
        kc, vc, L0 = caches[layer]
        out, ao, sel, gates, k, v = onb.block_step(want, W, kc, vc, L0, window, rope, cos, sin, CFG, experts)
        kc[:, L0], vc[:, L0] = k, v
        want = out
        cold = bank.begin_moe_layer(layer, hs["gain"], hs["router"], hs["wq"], hs["wk"], hs["wv"], hs["wo"], state,
                                    FW, 1, window, rope)
        bound = {0} if layer == 1 else set()
        expect_cold = [int(e) for e in dict.fromkeys(sel.tolist()) if int(e) not in bound]
        assert list(cold) == expect_cold
        if layer == 0 and cold:                         # continuing with a cold expert unbound fails closed (rc 4)
            with pytest.raises(qk_gpu.CudaContextError):
                bank.continue_moe_layer(layer, FW)
        for e in cold:
            bank.bind_moe_expert(layer, e, *eh[e])
        state = bank.continue_moe_layer(layer, FW, publish=layer == 1)
    assert np.array_equal(state, want)
    assert np.array_equal(bank.export_moe_hidden(), want)
    bank.reset()
    assert bank.length(0) == 0
    bank.close()
    qk_gpu.free_all()


def test_bank_guard_poisons_layer(gpu):
    from integer_inference_engine_amd import qk_gpu
    W, hs, _, _ = _weights(9)
    cos, sin = build_rope_tables(CAP, HD, base=50000, frac=FA)
    bank = qk_gpu.ResidentAttentionCache(1, CAP, D, H, HKV, HD, FA, cos, sin)
    huge = np.full((1, D), 1 << 50, dtype=np.int64)     # q . k leaves int64
    with pytest.raises(qk_gpu.CudaContextError):
        bank.apply(0, hs["wq"], hs["wk"], hs["wv"], hs["wo"], huge, FW, None, True)
    with pytest.raises(qk_gpu.CudaContextError):        # the poisoned layer refuses further work
        bank.apply(0, hs["wq"], hs["wk"], hs["wv"], hs["wo"], np.zeros((1, D), np.int64), FW, None, False)
    bank.close()
    qk_gpu.free_all()


def test_token_executor_chains_layers_like_the_oracle(gpu):
    """ResidentMoeTokenExecutor (qk_cuda.py:738-868): two consecutive layers with one expert resident up front
    (lookup) and the rest loaded lazily on the device's cold report; result equals two oracle block steps. A bad
    loader poisons the executor."""
    from integer_inference_engine_amd import qk_gpu
    W, hs, experts, eh = _weights(17)
    cos, sin = build_rope_tables(CAP, HD, base=50000, frac=FA)
    bank = qk_gpu.ResidentAttentionCache(2, CAP, D, H, HKV, HD, FA, cos, sin)
    rng = np.random.default_rng(18)
    caches = []
    for layer in range(2):
        L0 = 4 + layer
        kc = np.zeros((HKV, CAP, HD), dtype=np.int64)
        vc = np.zeros_like(kc)
        kc[:, :L0] = rng.integers(-(1 << 17), 1 << 17, size=(HKV, L0, HD))
        vc[:, :L0] = rng.integers(-(1 << 17), 1 << 17, size=(HKV, L0, HD))
        bank.import_layer(layer, kc[:, :L0], vc[:, :L0])
        caches.append([kc, vc, L0])
    loaded = []
    ex = qk_gpu.ResidentMoeTokenExecutor(
        bank, first_layer=0, layer_count=2, n_experts=E, n_used=USED, d_model=D, expert_ffn=EFF, fw=FW, eps=1,
        lookup_expert=lambda layer, e: eh[e] if (layer, e) == (1, 0) else None,
        load_expert=lambda layer, e: loaded.append((layer, e)) or eh[e])
    specs = [qk_gpu.ResidentMoeLayerSpec(l, hs["gain"], hs["router"], hs["wq"], hs["wk"], hs["wv"], hs["wo"],
                                         w, r) for l, (w, r) in enumerate([(None, False), (4, True)])]
    x = rng.integers(-(1 << 20), 1 << 20, size=(1, D), dtype=np.int64)
    got = ex.run(x, specs)
    want = x
    for layer, (window, rope) in enumerate([(None, False), (4, True)]):
        kc, vc, L0 = caches[layer]
        want, _, sel, _, k, v = onb.block_step(want, W, kc, vc, L0, window, rope, cos, sin, CFG, experts)
    assert np.array_equal(got, want)
    assert (1, 0) not in loaded and loaded                 # the resident one was bound, the others loaded lazily
    bank.reset()
    bank2 = qk_gpu.ResidentAttentionCache(1, CAP, D, H, HKV, HD, FA, cos, sin)
    bad = qk_gpu.ResidentMoeTokenExecutor(
        bank2, first_layer=0, layer_count=1, n_experts=E, n_used=USED, d_model=D, expert_ffn=EFF, fw=FW, eps=1,
        lookup_expert=lambda layer, e: None, load_expert=lambda layer, e: (1, 2))
    with pytest.raises(qk_gpu.CudaContextError):
        bad.run(x, specs[:1])
    assert bad.poisoned
    with pytest.raises(qk_gpu.CudaContextError):
        bad.run(x, specs[:1])
    bank2.close()
    bank.close()
    qk_gpu.free_all()
