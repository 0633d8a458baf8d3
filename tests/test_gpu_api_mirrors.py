"""Reference producer entry points mirrored for drop-in use (gpu_native.py:334-361, qk_cuda.py:24-34, 319-330,
870-910, 1029-1101): failure-atomic reservations, boundary telemetry, capability probes, the Q6_K DP4A alias."""
import numpy as np
import pytest

from oracle import qk

pytestmark = pytest.mark.gpu


def test_gpu_reservations_are_failure_atomic(gpu):
    before = gpu.gpu_memory_info()["free_bytes"]
    got = gpu.gpu_reservation_create([1 << 20, 3 << 20])
    assert got is not None and got[1] == 4 << 20
    assert gpu.gpu_memory_info()["free_bytes"] <= before - (4 << 20)
    gpu.gpu_reservation_free(got[0])
    gpu.gpu_reservation_free(got[0])                   # second free is a no-op
    assert gpu.gpu_reservation_create([1 << 20, 1 << 50]) is None       # cannot fit: nothing left behind
    assert gpu.gpu_memory_info()["free_bytes"] >= before - (64 << 20)
    with pytest.raises(ValueError):
        gpu.gpu_reservation_create([1 << 20, 0])


def test_qk_telemetry_probes_and_q6k_dp4a_alias(gpu):
    from integer_inference_engine_amd import qk_gpu
    assert qk_gpu.resident_preprocess_available()
    assert qk_gpu.moe_ffn_dp4a_available() and qk_gpu.moe_ffn_batched_dp4a_available()
    assert qk_gpu.resident_preprocess_bytes(2, 256, 8) == 2 * 9 * 256 * 8
    with pytest.raises(ValueError):
        qk_gpu.resident_preprocess_bytes(1, 0, 8)
    assert qk_gpu.profile_reset(enabled=True)
    raw = qk.random_blocks(3, 0, 48, 2, 1)
    h = qk_gpu.register_weight(raw, 48, 2, 1)
    x = np.random.default_rng(4).integers(-(1 << 18), 1 << 18, size=(2, 512), dtype=np.int64)
    want = qk.linear(x, qk.dequant(raw, 48, 2, 1, 24), 24)
    assert np.array_equal(qk_gpu.apply_resident(h, x, 48, 24), want)
    assert np.array_equal(qk_gpu.apply_resident_q6k_dp4a(h, x, 48, 24), want)
    snap = qk_gpu.profile_snapshot()
    assert set(snap) == set(qk_gpu.PROFILE_METRICS)
    assert snap["registration_calls"] >= 1 and snap["resident_apply_calls"] >= 1
    assert qk_gpu.profile_set_enabled(False)
    assert isinstance(qk_gpu.moe_workspace_allocations(), int)
    qk_gpu.free_all()
