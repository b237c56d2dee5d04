"""Host-side sanitizer build of libdizo_amd.so (CPU only; no GPU run loads it).

The C ABI's host code (argument and range checks, table construction, the
quantile table, the allocation-free entry point's plan batching) is compiled
with AddressSanitizer and UndefinedBehaviorSanitizer; the device code is
compiled as in the product build (every -fsanitize= flag applies to the host
compilation only, through -Xarch_host). The result goes to
dizo_amd/_sanitized/libdizo_amd.so, apart from the product library.

A process that loads it needs the clang AddressSanitizer runtime first (the
Python interpreter is not instrumented): run_tests() starts pytest in a child
process with that runtime preloaded and DIZO_AMD_LIB pointing at the build,
and returns its exit status.

Usage: python -m dizo_amd.build_sanitized [pytest arguments]
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys

from . import build as B

OUT = os.path.join(B.PKG_DIR, "_sanitized", "libdizo_amd.so")
HOST_SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                 "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer",
                 "-Xarch_host", "-g"]


def asan_runtime() -> str:
    """The clang AddressSanitizer shared runtime of the ROCm toolchain."""
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    hits = sorted(glob.glob(os.path.join(rocm, "lib", "llvm", "lib", "clang", "*", "lib", "linux",
                                         "libclang_rt.asan-x86_64.so")))
    if not hits:
        raise RuntimeError("libclang_rt.asan-x86_64.so not found under the ROCm LLVM")
    return hits[-1]


def build(verbose: bool = False) -> str:
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    return B.build(verbose=verbose, out=OUT, extra_flags=HOST_SANITIZE)


def run_tests(pytest_args, lib: str = OUT) -> int:
    env = dict(os.environ)
    env["LD_PRELOAD"] = asan_runtime()
    env["DIZO_AMD_LIB"] = lib
    # the interpreter's own allocations are not freed at exit: leaks are not reported
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0:halt_on_error=1:exitcode=86"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1:exitcode=87"
    return subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", *pytest_args],
                          env=env, cwd=os.path.dirname(B.PKG_DIR)).returncode


if __name__ == "__main__":
    print(build(verbose=True), flush=True)
    sys.exit(run_tests(sys.argv[1:] or ["tests/test_abi.py", "tests/test_c_consumer.py",
                                        "tests/test_abi_errors.py"]))
