"""A non-Python host of the C ABI: a C99 program compiled with gcc against
include/dizo_amd.h and linked with libdizo_amd.so calls the host-side entry
points (no GPU): the version, a block of the z generator (Philox4x32-7) and the
quantile table.
Its output matches the oracle."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from dizo_amd import _lib as L
from oracle import rng

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROGRAM = r"""
#include <stdio.h>
#include <inttypes.h>
#include "dizo_amd.h"

int main(void) {
  uint32_t block[4];
  uint16_t table[32768];
  printf("version %d\n", (int)dz_version());
  if (dz_philox_host(123456789ull, DZ_STREAM_PARAM, 77ull, block) != DZ_OK) {
    printf("error %s\n", dz_last_error());
    return 1;
  }
  printf("philox %" PRIu32 " %" PRIu32 " %" PRIu32 " %" PRIu32 "\n", block[0], block[1], block[2], block[3]);
  if (dz_normal_table(DZ_DTYPE_F16, table, 32768) != DZ_OK) {
    printf("error %s\n", dz_last_error());
    return 1;
  }
  printf("table %u %u %u\n", (unsigned)table[0], (unsigned)table[16384], (unsigned)table[32767]);
  /* an invalid call reports an error code and a message instead of aborting */
  int32_t rc = dz_normal_table(99, table, 32768);
  printf("bad %d %s\n", (int)rc, rc < 0 ? "message" : "none");
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no gcc")
def test_c_program_uses_the_abi(tmp_path):
    lib = L.lib_path()
    if not os.path.exists(lib):
        pytest.skip("library not built")
    src = tmp_path / "consumer.c"
    src.write_text(PROGRAM)
    exe = tmp_path / "consumer"
    libdir = os.path.dirname(lib)
    # --allow-shlib-undefined: the host-sanitizer build of the library
    # (dizo_amd.build_sanitized) takes its sanitizer runtime from the process
    # that loads it
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src),
                    "-o", str(exe), lib, f"-Wl,-rpath,{libdir}", "-Wl,--allow-shlib-undefined"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    assert out[0] == f"version {L.load().dz_version()}"
    want = rng.philox_groups(123456789, 0, [77])[0]
    assert out[1] == "philox " + " ".join(str(int(x)) for x in want)
    q = rng.quantile_table("f16")
    assert out[2] == f"table {int(q[0])} {int(q[16384])} {int(q[32767])}"
    assert out[3].startswith("bad -") and out[3].endswith("message")
