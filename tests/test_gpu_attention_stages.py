"""Stage-level checks of the attention pipeline (scores, softmax probabilities, PV accumulator) vs numpy."""
import numpy as np
import pytest

from oracle import fixedpoint as fx, prng, workloads

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("stage", [1, 2, 3])
def test_attention_stages(gpu, stage):
    from integer_inference_engine_amd import _lib
    so = _lib.lib()
    H, Hkv, hd, M, start = 4, 2, 32, 5, 0
    L = start + M
    q = prng.uniform_int(3, 1, (H, M, hd), -(1 << 20), 1 << 20)
    k, _ = workloads.kv_fill(3, 2, Hkv, L, hd)
    sc = np.zeros((H * M, L), dtype=np.int64)
    rm = np.zeros(H * M, dtype=np.int64)
    acc = np.zeros((H * M, hd), dtype=np.int64)
    assert so.imie_attention_scores_probe(q.ctypes.data, k.ctypes.data, H, Hkv, hd, M, L, start, 16, 11585,
                                          sc.ctypes.data, rm.ctypes.data, stage, acc.ctypes.data) == 0
    rep = H // Hkv
    for h in range(H):
        for m in range(M):
            s = ((q[h, m] @ k[h // rep, :m + 1].T) >> 16)
            s = (s * 11585) >> 16
            r = h * M + m
            assert rm[r] == s.max(), (h, m, rm[r], s.max())
            p = fx.softmax_rows(s[None], 16)[0]
            if stage == 1:
                assert list(sc[r, :m + 1]) == list(s), (h, m, sc[r, :m + 1], s)
            else:
                assert list(sc[r, :m + 1]) == list(p), (h, m, sc[r, :m + 1], p)
            if stage == 3:
                assert list(acc[r]) == list(p @ k[h // rep, :m + 1]), (h, m)
