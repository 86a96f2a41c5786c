"""Build libqmm.so (HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

    python mlx-runner_amd/build.py          # compile every source, link libqmm.so

Objects go to mlx-runner_amd/_build/, the library to mlx-runner_amd/libqmm.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libqmm.so"
SOURCES = ["qmv.hip", "qmv_mfma.hip", "gdn.hip", "gdn_chunk.hip", "gemm.hip", "gemm_fp8.hip", "gemm_nvfp4.hip", "quant.hip", "qmm_api.cpp", "weights.cpp", "checkpoint.cpp"]
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    # packed FP32 ops stay disabled on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Decode kernels (GEMVs, the GDN step): the leading kernel arguments (sizes and pointers,
# up to 16 dwords) arrive preloaded in SGPRs, so a wave issues its first loads without a
# kernel-argument round trip (gfx950 firmware; the code keeps a loading prologue for
# firmware without it).
PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=16"]
EXTRA = {"qmv_mfma.hip": PRELOAD, "qmv.hip": PRELOAD, "gdn.hip": PRELOAD}


def _compile(src: str) -> Path:
    obj = BUILD / (src + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-I", str(HERE.parent / "include"), "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msgs}")
    if msgs.strip():
        print(msgs, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
