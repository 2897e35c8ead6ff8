"""Builds ``libcchip.so`` (the runtime + Backend_hip C-ABI) in-tree.

The library is host code over the HIP runtime and hiprtc; the kernels it
runs are generated per graph and compiled by hiprtc for gfx950 at
``compile`` time. ``check_templates`` JIT-compiles a representative set of
generated modules without a GPU, so template errors surface at build time.
"""

from __future__ import annotations

import glob
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libcchip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def build(verbose=False):
    srcs = sorted(glob.glob(os.path.join(HERE, "csrc", "*.cpp")))
    tmp = LIB + ".tmp%d" % os.getpid()
    cmd = [
        os.path.join(ROCM, "bin", "hipcc"),
        "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-D__HIP_PLATFORM_AMD__",
        "-I" + os.path.join(ROCM, "include"),
        "-o", tmp,
    ] + srcs + [
        "-L" + os.path.join(ROCM, "lib"), "-Wl,-rpath," + os.path.join(ROCM, "lib"),
        "-lhiprtc", "-lamdhip64",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
