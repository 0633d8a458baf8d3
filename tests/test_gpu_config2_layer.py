"""Config 2: one Bonsai-8B-shape decoder layer, decode at batch 1 over a 4096-token int32 paged KV cache.
Layer output and the new KV entries must equal the oracle byte for byte."""
import numpy as np
import pytest

from oracle import bonsai_model as obm, c_oracle, prng, workloads
from oracle.rope import bonsai8b_tables
from tests.bonsai_gpu_harness import register_model

pytestmark = pytest.mark.gpu

D, H, HKV, HD, DFF, CTX = 4096, 32, 8, 128, 12288, 4096


def _model():
    layer = workloads.bonsai_layer(2, D, H, HKV, HD, DFF)
    cos, sin = bonsai8b_tables(CTX + 8)
    return {"layers": [layer], "cos": cos, "sin": sin}


@pytest.mark.parametrize("page", [64, 4096 + 64])
def test_config2_layer_decode_byte_exact(gpu, page):
    import torch
    from integer_inference_engine_amd.resident import ResidentNet
    model = _model()
    w, g = register_model(gpu, model, with_head=False)
    kc, vc = workloads.kv_fill(2, 50, HKV, CTX, HD)
    x_in = prng.uniform_int(2, 60, (1, D), -(1 << 20), 1 << 20)
    net = ResidentNet(B=1, n_layers=1, H=H, Hkv=HKV, hd=HD, d=D, dff=DFF, cap=CTX + 8, w=w, g=g, page=page, kv32=True)
    net.seed(0, kc[None], vc[None])
    x = torch.from_numpy(x_in.copy()).cuda()
    status = net.forward(x, [CTX], 1)
    assert status == 0
    got_x = x.cpu().numpy()
    got_k, got_v = net.export_kv(0, 0, CTX + 1)
    net.close()
    c = {"H": H, "Hkv": HKV, "hd": HD}
    want_x, kn, vn = obm.layer_forward(x_in, model["layers"][0], c, model["cos"], model["sin"], 16, kc, vc, CTX,
                                       q1=c_oracle.q1_linear)
    assert np.array_equal(got_k[:, :CTX], kc) and np.array_equal(got_v[:, :CTX], vc)
    assert np.array_equal(got_k[:, CTX:], kn), "new K row"
    assert np.array_equal(got_v[:, CTX:], vn), "new V row"
    assert np.array_equal(got_x, want_x), f"{np.count_nonzero(got_x != want_x)} residual mismatches"
