"""Builds libaffx.so (gfx950) in-tree with hipcc.

The library is plain HIP C++ behind the C-ABI of include/affx.h; Python reaches it through
ctypes (affinity_amd/_lib.py). Built in-tree so the .so travels with the source tree.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libaffx.so")
SOURCES = ["affx_layout.hip", "affx_decode.hip", "affx_fused.hip", "affx_quant.hip", "affx_grouped.hip", "affx_api.hip",
           "affx_noalloc.hip", "affx_route.hip", "affx_shared.hip", "affx_fit.hip", "affx_gemv.hip", "affx_steps.hip", "affx_w8a8.hip",
           "affx_container.cpp", "affx_blas.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 anywhere in device code (hipcc's host pass warns
# that it does not know the feature; the device pass honours it).
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-command-line-argument"]
# hipBLASLt for the shared expert's batch GEMMs (affx_blas.cpp); in a process that has loaded
# torch first, the dynamic loader resolves it to the copy torch already holds
LIBS = ["-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib"]


def build(verbose: bool = False) -> str:
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *FLAGS, *srcs, "-o", tmp, *LIBS]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed:\n{' '.join(cmd)}\n{msgs}")
    if verbose and msgs.strip():
        print(msgs)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
