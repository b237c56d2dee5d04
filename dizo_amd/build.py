"""Builds libdizo_amd.so (HIP, gfx950) in-tree with hipcc.

Usage: ``python -m dizo_amd.build`` or ``dizo_amd.build.build()``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_PATH = os.path.join(PKG_DIR, "libdizo_amd.so")
SOURCES = ["dz_kernels.hip", "dz_api.hip"]
HEADERS = ["dz_common.h", "dz_kernels.h"]

# -ffp-contract=off: products must not be contracted into FMAs (bit parity with
# PyTorch's one-rounding-per-op recipe). -packed-fp32-ops: no v_pk_*_f32.
# -amdgpu-atomic-optimizer-strategy=None: the kernels' work-counter atomics
# run on one lane; the optimizer's wave-wide rewrite of them only adds a
# readfirstlane of the result and a wait for it right after the atomic
# (measured: perturb and update passes 0.7-2.3 % faster without it).
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False, out: str = LIB_PATH, extra_flags=()) -> str:
    """Compiles the library (always; no up-to-date check) and returns its path."""
    tmp = out + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, *extra_flags, *[os.path.join(CSRC, s) for s in SOURCES], "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l and l.strip())
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err:
        print(err, file=sys.stderr)
    os.replace(tmp, out)
    return out


C_HOST_SRC = os.path.join(CSRC, "zo_step_host.c")
C_HOST_PATH = os.path.join(os.path.dirname(LIB_PATH), "zo_step_host")


def build_c_host(verbose: bool = False, lib: str = LIB_PATH, out: str = C_HOST_PATH) -> str:
    """Compiles csrc/zo_step_host.c, a C99 host of the ZO step through the C ABI
    (gcc, HIP runtime C API, linked with the library), and returns its path."""
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    include = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    libdir = os.path.dirname(os.path.abspath(lib))
    cmd = ["gcc", "-std=c99", "-O2", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
           "-I", include, "-I", os.path.join(rocm, "include"), C_HOST_SRC, "-o", out + ".tmp",
           "-L", libdir, "-ldizo_amd", "-Wl,-rpath,$ORIGIN", "-L", os.path.join(rocm, "lib"), "-lamdhip64",
           f"-Wl,-rpath,{os.path.join(rocm, 'lib')}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed ({res.returncode}):\n{res.stderr}")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_c_host(verbose=True))
