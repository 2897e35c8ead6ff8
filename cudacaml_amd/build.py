"""Builds ``libcchip.so`` (the runtime + Backend_hip C-ABI) in-tree.

The library is host code over the HIP runtime and hiprtc; the kernels it
runs are generated per graph and compiled by hiprtc for gfx950 at
``compile`` time. Its own device code (``csrc/*.hip``, built for gfx950
here) is the static scratch of the allocation-free entry point and the
kernel that clears it. ``check_templates`` JIT-compiles a representative set of
generated modules without a GPU, so template errors surface at build time.
"""

from __future__ import annotations

import glob
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libcchip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


ASAN_LIB = os.path.join(HERE, "libcchip_asan.so")
ASAN_RUNTIME = os.path.join(ROCM, "llvm", "lib", "clang", "*", "lib", "linux", "libclang_rt.asan-x86_64.so")


def build(verbose=False, asan=False):
    """``asan=True`` builds ``libcchip_asan.so`` with AddressSanitizer on
    the host code only (the generated kernels are compiled by hiprtc at run
    time; the library's own device code is one fill kernel and the static
    scratch array of the allocation-free entry point). It is for CPU runs: load it with
    ``CCHIP_LIB`` pointing at it and the sanitizer runtime preloaded (see
    ``asan_env``)."""
    srcs = sorted(glob.glob(os.path.join(HERE, "csrc", "*.cpp"))) + sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")))
    out = ASAN_LIB if asan else LIB
    tmp = out + ".tmp%d" % os.getpid()
    cmd = [
        os.path.join(ROCM, "bin", "hipcc"),
        "--offload-arch=gfx950", "-O1" if asan else "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
        "-Wno-unused-function",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-D__HIP_PLATFORM_AMD__",
        "-I" + os.path.join(ROCM, "include"),
    ]
    if asan:
        cmd += ["-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]
    cmd += ["-o", tmp] + srcs + [
        "-L" + os.path.join(ROCM, "lib"), "-Wl,-rpath," + os.path.join(ROCM, "lib"),
        "-lhiprtc", "-lamdhip64",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


def asan_env():
    """Environment for a CPU test run against ``libcchip_asan.so``."""
    rt = sorted(glob.glob(ASAN_RUNTIME))
    if not rt:
        raise FileNotFoundError("no AddressSanitizer runtime under " + ASAN_RUNTIME)
    env = dict(os.environ)
    env.update(CCHIP_LIB=ASAN_LIB, LD_PRELOAD=rt[-1], ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    return env


if __name__ == "__main__":
    import sys

    if "--asan-tests" in sys.argv:
        # python -m cudacaml_amd.build --asan-tests: the CPU suite against
        # the host-sanitized library
        build(verbose=True, asan=True)
        rc = subprocess.run([sys.executable, "-m", "pytest", os.path.join(os.path.dirname(HERE), "tests"), "-m",
                             "not gpu", "-x", "-q", "-p", "no:cacheprovider"], env=asan_env()).returncode
        sys.exit(rc)
    build(verbose=True, asan="--asan" in sys.argv)
