"""GGUF-imported weights registered in the resident managers and applied on the device, against the oracle on the
same imported integers (the reference's import -> register path: import_bonsai_gguf.py:17-93 feeding
gpu_native.py:270-306, nmc/gguf.py:108-113 feeding qk_cuda.py:252-270)."""
import numpy as np
import pytest

from integer_inference_engine_amd import gguf
from oracle import qk
from oracle.q1 import q1_linear
from tests.gguf_writer import _q1_blocks, write_gguf

pytestmark = pytest.mark.gpu


def test_imported_q1_and_expert_apply_on_device(gpu, tmp_path):
    from integer_inference_engine_amd import qk_gpu
    rng = np.random.default_rng(21)
    out_f, nb = 96, 4
    sc = (rng.standard_normal(out_f * nb) * 0.02).astype(np.float16)
    blocks = _q1_blocks(rng, out_f, nb, sc)
    n_e, eo, ein = 3, 64, 512
    e_raw = [qk.random_blocks(22, e, eo, ein // 256, 0) for e in range(n_e)]
    p = tmp_path / "m.gguf"
    write_gguf(p, [], [("blk.0.ffn_up.weight", [nb * 128, out_f], gguf.Q1_0, blocks.tobytes()),
                       ("blk.0.ffn_up_exps.weight", [ein, eo, n_e], gguf.Q4_K, b"".join(r.tobytes() for r in e_raw))])
    g = gguf.GGUF(p)
    hs = gguf.register_q1(g, ["blk.0.ffn_up.weight"], 16)
    bits, scale = g.q1_packed("blk.0.ffn_up.weight", 16)
    x = rng.integers(-(1 << 18), 1 << 18, size=(3, nb * 128), dtype=np.int64)
    got = gpu.q1_apply_resident(hs["blk.0.ffn_up.weight"], x, out_f, nb, 16)
    assert np.array_equal(got, q1_linear(x, bits, scale, 16))
    xe = rng.integers(-(1 << 18), 1 << 18, size=(2, ein), dtype=np.int64)
    for e in range(n_e):
        h = gguf.register_expert(g, "blk.0.ffn_up_exps.weight", e)
        want = qk.linear(xe, qk.dequant(e_raw[e], eo, ein // 256, 0, 24), 24)
        assert np.array_equal(qk_gpu.apply_resident(h, xe, eo, 24), want), e
    gpu.q1_free_weights()
    qk_gpu.free_all()


def test_artifact_from_gguf_prefills_on_device_like_the_oracle(gpu, tmp_path):
    """GGUF -> artifact -> safetensors -> load -> register_artifact -> device prefill logits and K/V, against the
    oracle forward of the same loaded artifact."""
    from integer_inference_engine_amd import artifact as A
    from oracle import bonsai_model as obm, fixedpoint as fx
    from oracle.q1 import q1_rows
    from tests.gguf_writer import artifact_model, bonsai_gguf
    src = tmp_path / "b.gguf"
    bonsai_gguf(src, seed=31)
    A.save(A.import_gguf(src), tmp_path / "b.safetensors", provenance=A.gguf_provenance(src))
    art, _ = A.load(tmp_path / "b.safetensors")
    dm = A.dims(art)
    w, g = A.register_artifact(art)
    model = artifact_model(art)
    c = {"H": dm["H"], "Hkv": dm["Hkv"], "hd": dm["hd"]}
    ids = np.random.default_rng(32).integers(0, dm["vocab"], size=9)
    x0 = q1_rows(*model["embed"], ids)
    dims = (len(ids), dm["d"], dm["n_layers"], dm["H"], dm["Hkv"], dm["hd"], dm["dff"])
    inv = fx.inv_sqrt_fp(dm["hd"], 16)
    logits, k, v = gpu.prefill_forward_gpu(x0, dims, w, g, 16, 1, inv, export_kv=True)
    x, ks, vs = x0, [], []
    for layer in model["layers"]:
        x, kn, vn = obm.layer_forward(x, layer, c, model["cos"], model["sin"], 16, None, None, 0)
        ks.append(kn)
        vs.append(vn)
    assert np.array_equal(logits, obm.head_logits(model, x[-1:], 16)[0])
    assert np.array_equal(k, np.stack(ks)) and np.array_equal(v, np.stack(vs))
    gpu.q1_free_weights()
