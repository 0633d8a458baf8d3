"""Register a synthetic Bonsai model on the device through the reference-shaped boundary (test helper)."""
from __future__ import annotations

import numpy as np

from oracle.workloads import PROJ


def register_model(gpu, model: dict, with_head: bool = True):
    """Returns (w, g) handle bundles in the reference's ``gpu_native`` format (gpu_native.py:483-595)."""
    w = {name: [] for name in PROJ}
    g = {name: [] for name in ("n1g", "n2g", "qng", "kng")}
    for layer in model["layers"]:
        for name in PROJ:
            h = gpu.q1_register_weight(*layer[name])
            assert h is not None
            w[name].append(h)
        for name in g:
            h = gpu.buf_upload_i64(layer[name])
            assert h is not None
            g[name].append(h)
    w = {k: np.array(v, dtype=np.int64) for k, v in w.items()}
    g = {k: np.array(v, dtype=np.int64) for k, v in g.items()}
    if with_head:
        w["out_head"] = gpu.q1_register_weight(*model["out"])
        w["out_head_vocab"] = int(model["out"][1].shape[0])
        g["finalg"] = gpu.buf_upload_i64(model["final_g"])
    else:
        w["out_head"] = -1
        w["out_head_vocab"] = 0
        g["finalg"] = -1
    g["cos_h"] = gpu.buf_upload_i64(model["cos"])
    g["sin_h"] = gpu.buf_upload_i64(model["sin"])
    return w, g
