"""The C ABI driven by a C99 program with no Python or torch
(dizo_amd/csrc/zo_step_host.c, built next to the library by build()): one ZO
step and the next step's first perturbation, then a projection norm and apply,
on hipMalloc'd fp16 buffers. Its output is compared with the oracle: the
tensors bit for bit, the sums of squares to fp64 rounding (the order of the
fp64 sum differs)."""
import os
import subprocess

import numpy as np
import pytest

from oracle import arith as A
from oracle import rng
from oracle.arith import F16

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "dizo_amd", "zo_step_host")
NUMEL = [70001, 32768, 5]


def _start_bits(t: int, n: int) -> np.ndarray:
    """start_bits() of the C program: ((i * 2654435761 + t * 40503) mod 2^32 >> 16) & 0xbfff."""
    i = np.arange(n, dtype=np.uint64)
    h = (i * np.uint64(2654435761) + np.uint64(t * 40503)) & np.uint64(0xFFFFFFFF)
    return ((h >> np.uint64(16)) & np.uint64(0xBFFF)).astype(np.uint16)


def test_c_host_runs_a_zo_step_and_a_projection(tmp_path):
    assert os.path.exists(EXE), "zo_step_host is not built (run __graft_entry__.build())"
    out = tmp_path / "out.bin"
    print(f"running {EXE}", flush=True)
    r = subprocess.run([EXE, str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "zo_step_host ok" in r.stdout
    raw = out.read_bytes()
    seed, seed2, eps, g, lr = 26, 27, 1e-3, -1.25, 1e-3
    offs = rng.layout_z_offsets(NUMEL)
    start = [_start_bits(t, n) for t, n in enumerate(NUMEL)]
    pos = 0
    after_zo = []
    for t, n in enumerate(NUMEL):
        got = np.frombuffer(raw[pos:pos + 2 * n], dtype=np.uint16)
        pos += 2 * n
        z = rng.tensor_z_bits(seed, offs[t], n, F16)
        z2 = rng.tensor_z_bits(seed2, offs[t], n, F16)
        h = A.perturb(A.perturb(start[t], z, 1, eps, F16), z, -2, eps, F16)
        want = A.perturb(A.restore_update(h, z, eps, g, lr, F16), z2, 1, eps, F16)
        np.testing.assert_array_equal(got, want, err_msg=f"ZO passes, tensor {t}")
        after_zo.append(want)
    sumsq = np.frombuffer(raw[pos:pos + 8 * len(NUMEL)], dtype=np.float64)
    pos += 8 * len(NUMEL)
    for t in range(len(NUMEL)):
        want = A.group_sumsq(after_zo[t], start[t], F16)
        assert sumsq[t] == pytest.approx(want, rel=1e-12), t
    alpha = np.array([0x3A00], dtype=np.uint16)  # 0.75
    for t, n in enumerate(NUMEL):
        got = np.frombuffer(raw[pos:pos + 2 * n], dtype=np.uint16)
        pos += 2 * n
        np.testing.assert_array_equal(got, A.apply(after_zo[t], start[t], alpha, F16), err_msg=f"apply, tensor {t}")
    assert pos == len(raw)
