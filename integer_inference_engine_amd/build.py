"""Build ``libimie_gfx950.so`` in-tree from ``csrc/*.hip`` with hipcc for gfx950.

``python -m integer_inference_engine_amd.build`` (or ``__graft_entry__.build()``) always recompiles. Objects are
compiled in parallel into ``_build/`` next to this file, then linked into one shared library whose C-ABI is
declared in ``include/imie_bonsai.h`` and ``include/imie_nmc.h``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libimie_gfx950.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # packed FP32 instructions are disabled for every HIP object (no packed-fp32 codegen on this pool)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the integer kernels rework every MFMA result with VALU ops (limb shifts,
    # recombination), which the AGPR form would route through v_accvgpr_read / write copies
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-result",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    if src.suffix == ".cpp":                          # host-only C++ (the CPU verifier): no device code
        cmd = [HIPCC, "-x", "c++", "-O3", "-fPIC", "-std=c++17", "-pthread", "-c", str(src), "-o", str(obj)]
    else:
        cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr[-4000:]}")
    return obj


def build(verbose: bool = False) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
