"""imie_q1_apply_dev_noalloc (the allocation-free variant of imie_q1_apply_dev, fixed device scratch) against
imie_q1_apply_dev and the oracle, through the C-ABI: two calls in a row, the second smaller, then the size
refusals. The scratch keeps the last call's contents, so the second call also shows nothing stale is read."""
import ctypes

import numpy as np
import pytest

from oracle import prng
from oracle.q1 import q1_linear

pytestmark = pytest.mark.gpu


def _apply(so, fn, h, x, N, frac):
    import torch
    xd = torch.from_numpy(x).cuda()
    out = torch.full((x.shape[0], N), -7, dtype=torch.int64, device="cuda")
    st = torch.cuda.current_stream()
    rc = fn(h, ctypes.c_void_p(xd.data_ptr()), x.shape[0], frac, ctypes.c_void_p(out.data_ptr()),
            ctypes.c_void_p(st.cuda_stream))
    st.synchronize()
    return rc, out.cpu().numpy()


def test_noalloc_matches_allocating_entry_point(gpu):
    from integer_inference_engine_amd import _lib
    so = _lib.lib()
    cases = [(12288, 96, 5, 1 << 40, 16), (4096, 32, 1, 127, 16)]     # second call: fewer tokens, shorter K
    for N, nb, T, mag, frac in cases:
        print(f"[noalloc] N={N} nb={nb} T={T}", flush=True)
        bits = prng.uniform_bytes(N + T, 1, (N, nb, 16))
        scale = prng.uniform_int(N + T, 2, (N, nb), -(1 << 20), 1 << 20)
        x = prng.uniform_int(N + T, 3, (T, nb * 128), -mag, mag + 1)
        h = gpu.q1_register_weight(bits, scale)
        assert h is not None
        rc0, want = _apply(so, so.imie_q1_apply_dev, h, x, N, frac)
        rc1, got = _apply(so, so.imie_q1_apply_dev_noalloc, h, x, N, frac)
        assert rc0 == 0 and rc1 == 0
        assert np.array_equal(got, want)
        assert np.array_equal(got, q1_linear(x, bits, scale, frac))


def test_noalloc_refuses_sizes_beyond_its_scratch(gpu):
    from integer_inference_engine_amd import _lib
    so = _lib.lib()
    bits = prng.uniform_bytes(3, 1, (16, 2, 16))
    scale = prng.uniform_int(3, 2, (16, 2), 1, 100)
    h = gpu.q1_register_weight(bits, scale)
    rc, _ = _apply(so, so.imie_q1_apply_dev_noalloc, h, prng.uniform_int(3, 3, (8, 256), -9, 9), 16, 16)
    assert rc == 1 and b"at most 7 tokens" in so.imie_last_error()
    wide = gpu.q1_register_weight(prng.uniform_bytes(4, 1, (16, 257, 16)), prng.uniform_int(4, 2, (16, 257), 1, 9))
    rc, _ = _apply(so, so.imie_q1_apply_dev_noalloc, wide, prng.uniform_int(4, 3, (1, 257 * 128), -9, 9), 16, 16)
    assert rc == 1


def _free_bytes(so):
    free, total = ctypes.c_uint64(0), ctypes.c_uint64(0)
    assert so.bonsai_gpu_mem_info(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_noalloc_allocates_nothing_and_replays_in_a_graph(gpu):
    """The entry point's contract: no device allocation (free bytes unchanged across a call on a fresh weight
    after the one-time symbol lookup) and usable under stream capture. The captured call is replayed three times
    with new activations written between replays (eager work and synchronisations in between), each replay
    checked against the oracle."""
    import torch
    from integer_inference_engine_amd import _lib
    so = _lib.lib()
    N, nb, T, frac = 4096, 32, 3, 16
    bits = prng.uniform_bytes(91, 1, (N, nb, 16))
    scale = prng.uniform_int(91, 2, (N, nb), -(1 << 20), 1 << 20)
    h = gpu.q1_register_weight(bits, scale)
    assert h is not None
    xs = [prng.uniform_int(91, 3 + i, (T, nb * 128), -(1 << 30), (1 << 30) + 1) for i in range(4)]
    xd = torch.from_numpy(xs[0]).cuda()
    out = torch.zeros((T, N), dtype=torch.int64, device="cuda")
    st = torch.cuda.current_stream()
    fn = so.imie_q1_apply_dev_noalloc
    args = lambda s: (h, ctypes.c_void_p(xd.data_ptr()), T, frac, ctypes.c_void_p(out.data_ptr()),
                      ctypes.c_void_p(s.cuda_stream))
    assert fn(*args(st)) == 0                          # warm: resolves this device's scratch address
    torch.cuda.synchronize()
    free0 = _free_bytes(so)
    assert fn(*args(st)) == 0
    torch.cuda.synchronize()
    assert _free_bytes(so) == free0, "the allocation-free entry point changed the device's free memory"
    assert np.array_equal(out.cpu().numpy(), q1_linear(xs[0], bits, scale, frac))

    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(st)
    with torch.cuda.stream(cap):
        g.capture_begin()
        rc = fn(*args(cap))
        g.capture_end()
    torch.cuda.synchronize()
    assert rc == 0
    for i in (1, 2, 3):
        print(f"[noalloc] graph replay {i}", flush=True)
        xd.copy_(torch.from_numpy(xs[i]))
        out.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), q1_linear(xs[i], bits, scale, frac)), f"replay {i}"
