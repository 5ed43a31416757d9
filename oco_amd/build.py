"""Build the gfx950 shared library liboco_hip.so in-tree with hipcc.

The analogue of the reference's build.rs (which compiles shaders/oco.metal
with xcrun metal, build.rs:14-23): every source under csrc/ is compiled for
gfx950 and linked into one shared library exporting include/oco_hip.h.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_obj")
LIB = os.path.join(HERE, "liboco_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["matvec.hip", "matvec_group.hip", "runtime.hip", "dequant.hip", "routing.hip", "experts.hip", "matmul.hip", "mxmatmul.hip", "moe_prefill.hip", "mx_experts.hip", "elementwise.hip", "gguf.cpp"]

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # Packed FP32 instructions stay off (the compiler would otherwise form
    # v_pk_* ops from float2 code); the host pass warns that it does not know
    # the feature, which is harmless.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc", "-Wno-unused-command-line-argument",
    # Leading scalar kernel arguments arrive preloaded in SGPRs instead of
    # being fetched from the kernarg segment at wave start.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    f"-I{os.path.join(HERE, '..', 'include')}",
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build_library(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    sources = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    jobs = min(len(sources), 8)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB + ".tmp"
    # hipBLASLt: the plain f16 GEMM of the dequantize-then-GEMM prefill path
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lhipblaslt"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build_library(verbose=True)
