"""The Bonsai entry points added for the reference loader (dp4a apply, coalesced / bmma registrations), the
decode graph after a workspace regrowth, and the RoPE-table position bound, on gfx950 against the oracle.

References: bonsai_q1_gpu.cu:2245-2300 (dp4a apply, its digit kernel :419-432 and L=4 guard :475-481),
:2350-2385 (layout registrations), gpu_native.py:226-306 (their Python callers), reference_bonsai.py:1110-1146
(the greedy cached loop a decode graph replays)."""
import numpy as np
import pytest

from oracle import bonsai_model as obm, prng, workloads
from oracle.q1 import argmax_lowest, q1_linear, q1_rows
from oracle.rope import bonsai8b_tables
from tests.bonsai_gpu_harness import register_model

pytestmark = pytest.mark.gpu


def _trunc_digits(x, L):
    """The low L balanced base-256 digits of each int64, recombined mod 2^64 (bonsai_q1_gpu.cu:419-432)."""
    out = np.empty_like(x)
    for i, v in enumerate(x.reshape(-1)):
        r, acc = int(v) & ((1 << 64) - 1), 0
        for l in range(L):
            lb = r & 0xFF
            d = lb - 256 if lb >= 128 else lb
            acc += d << (8 * l)
            r = ((r - d) & ((1 << 64) - 1)) >> 8
        acc &= (1 << 64) - 1
        out.reshape(-1)[i] = acc - (1 << 64) if acc >= (1 << 63) else acc
    return out


@pytest.mark.parametrize("L", [4, -4, 8, -8, 3, 1])
def test_dp4a_apply_matches_oracle(gpu, L):
    from integer_inference_engine_amd import _lib
    so = _lib.lib()
    N, nb, T = 96, 5, 3
    bits = prng.uniform_bytes(77, 1, (N, nb, 16))
    scale = prng.uniform_int(77, 2, (N, nb), -(1 << 30), 1 << 30)
    cap = 127 * ((1 << (8 * min(abs(L), 7))) - 1) // 255
    x = prng.uniform_int(77, 3, (T, nb * 128), -min(cap, 1 << 40), min(cap, 1 << 40) + 1)
    if abs(L) < 4:                                        # values beyond L digits: the low-digit truncation
        x[0, :7] = [1 << 40, -(1 << 40), (1 << 62) + 5, -(1 << 63), (1 << 63) - 1, 300, -300]
        want = q1_linear(_trunc_digits(x, abs(L)), bits, scale, 16)
    else:
        want = q1_linear(x, bits, scale, 16)
    out = np.zeros((T, N), dtype=np.int64)
    rc = so.bonsai_q1_linear_dp4a_gpu(x.ctypes.data, bits.ctypes.data, scale.ctypes.data, T, N, nb, 16, L,
                                      out.ctypes.data)
    assert rc == 0 and np.array_equal(out, want)


def test_dp4a_l4_guard_and_mirror(gpu):
    from integer_inference_engine_amd import _lib
    so = _lib.lib()
    N, nb = 16, 2
    bits = prng.uniform_bytes(5, 1, (N, nb, 16))
    scale = prng.uniform_int(5, 2, (N, nb), -(1 << 11), 1 << 11)
    x = prng.uniform_int(5, 3, (2, nb * 128), -1000, 1000)
    x[1, 3] = 2139062144                                  # one past the L=4 guard
    out = np.zeros((2, N), dtype=np.int64)
    assert so.bonsai_q1_linear_dp4a_gpu(x.ctypes.data, bits.ctypes.data, scale.ctypes.data, 2, N, nb, 16, 4,
                                        out.ctypes.data) == 4
    with pytest.raises(ValueError, match="explicit L=4"):
        gpu.q1_apply_dp4a_gpu(x, bits, scale, 16, L=4)
    assert np.array_equal(gpu.q1_apply_dp4a_gpu(x, bits, scale, 16), q1_linear(x, bits, scale, 16))   # auto: L=8
    x[1, 3] = 7
    assert np.array_equal(gpu.q1_apply_dp4a_gpu(x, bits, scale, 16, L=4), q1_linear(x, bits, scale, 16))


@pytest.mark.parametrize("layout", ["gpu_coalesced", "gpu_bmma"])
def test_layout_registrations_apply_exactly(gpu, layout):
    N, nb = 72, 3
    bits = prng.uniform_bytes(9, 1, (N, nb, 16))
    scale = prng.uniform_int(9, 2, (N, nb), -(1 << 20), 1 << 20).astype(np.int32)
    x = prng.uniform_int(9, 3, (4, nb * 128), -(1 << 24), 1 << 24)
    with pytest.raises(ValueError, match="int32 scales"):
        gpu.q1_register_weight(bits, scale.astype(np.int64), **{layout: True})
    h = gpu.q1_register_weight(bits, scale, **{layout: True})
    assert h is not None
    got = gpu.q1_apply_resident(h, x, N, nb, 16)
    assert np.array_equal(got, q1_linear(x, bits, scale.astype(np.int64), 16))
    if layout == "gpu_bmma":                              # out_features % 8 != 0 is refused, as in the reference
        assert gpu.q1_register_weight(bits[:70], scale[:70], gpu_bmma=True) is None


D, H, HKV, HD, DFF, VOCAB = 256, 2, 1, 128, 384, 512
CFG = {"H": H, "Hkv": HKV, "hd": HD}


def _small_model(ctx, n_layers=2, seed=31):
    cos, sin = bonsai8b_tables(ctx)
    return {"layers": [workloads.bonsai_layer(seed, D, H, HKV, HD, DFF, li) for li in range(n_layers)],
            "cos": cos, "sin": sin, "embed": workloads.q1_weight(seed, 7, VOCAB, D),
            "out": workloads.q1_weight(seed, 9, VOCAB, D),
            "final_g": prng.uniform_int(seed, 11, (D,), 1 << 15, (1 << 17) + 1)}


def _oracle_greedy(model, prompt, steps):
    seq = list(prompt)
    for _ in range(steps):
        x = q1_rows(*model["embed"], np.array(seq))
        for layer in model["layers"]:
            x = obm.layer_forward(x, layer, CFG, model["cos"], model["sin"], 16, None, None, 0)[0]
        seq.append(int(argmax_lowest(obm.head_logits(model, x, 16)[-1:])[0]))
    return seq[len(prompt):]


def _replay(net, model, eb, es, prompt, steps):
    """Cached replay: prefill prompt[:-1], then the device greedy loop from prompt[-1] (graph-replayed)."""
    import torch
    net.reset()
    x = torch.from_numpy(q1_rows(*model["embed"], np.array(prompt[:-1]))).cuda()
    assert net.forward(x, [0], len(prompt) - 1) == 0
    ids = torch.tensor([prompt[-1]], dtype=torch.int64, device="cuda")
    _, hist = net.decode(eb, es, ids, steps, graph=True)
    net.stream.synchronize()
    return [int(t) for t in hist.cpu().numpy()[:, 0]]


def test_decode_graph_recaptured_after_workspace_regrowth(gpu):
    """A decode graph captured after a short prefill must not be replayed after a longer prefill has regrown (freed
    and reallocated) the workspaces it points into: short replay, long replay, short again, each equal to the
    oracle's greedy continuation."""
    import torch
    from integer_inference_engine_amd.resident import ResidentNet
    model = _small_model(128)
    w, g = register_model(gpu, model, with_head=True)
    net = ResidentNet(B=1, n_layers=2, H=H, Hkv=HKV, hd=HD, d=D, dff=DFF, cap=128, w=w, g=g, page=64, kv32=True)
    eb = torch.from_numpy(np.ascontiguousarray(model["embed"][0])).cuda()
    es = torch.from_numpy(np.ascontiguousarray(model["embed"][1])).cuda()
    try:
        short = [3, 9, 27]
        long = [int(v) for v in prng.uniform_int(4, 1, (90,), 0, VOCAB)]
        steps = 5
        for prompt in (short, long, short):
            assert _replay(net, model, eb, es, prompt, steps) == _oracle_greedy(model, prompt, steps), len(prompt)
    finally:
        net.close()


def test_positions_past_the_rope_table_are_refused(gpu):
    """Page rounding gives a sequence 128 slots from a 100-row RoPE table: positions 100.. must be refused
    (they would read past the uploaded table), and so must a capacity beyond the table."""
    import torch
    from integer_inference_engine_amd.resident import ResidentNet
    model = _small_model(100, n_layers=1)
    w, g = register_model(gpu, model, with_head=True)
    net = ResidentNet(B=1, n_layers=1, H=H, Hkv=HKV, hd=HD, d=D, dff=DFF, cap=100, w=w, g=g, page=64, kv32=True)
    eb = torch.from_numpy(np.ascontiguousarray(model["embed"][0])).cuda()
    es = torch.from_numpy(np.ascontiguousarray(model["embed"][1])).cuda()
    try:
        with pytest.raises(RuntimeError, match="set_caps"):
            net.set_caps([101])
        x = torch.from_numpy(q1_rows(*model["embed"], np.arange(98) % VOCAB)).cuda()
        assert net.forward(x, [0], 98) == 0
        with pytest.raises(RuntimeError, match="forward"):
            net.forward(x[:3].clone(), [98], 3)           # positions 98..100: 100 is past the table
        ids = torch.tensor([5], dtype=torch.int64, device="cuda")
        with pytest.raises(RuntimeError, match="decode"):
            net.decode(eb, es, ids, 3, graph=False)       # positions 98, 99, 100
        net.decode(eb, es, ids, 2, graph=False)           # 98 and 99 are still fine
        with pytest.raises(RuntimeError, match="fill_kv"):
            net.fill_kv(1, [101])
    finally:
        net.close()
