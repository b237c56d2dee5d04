"""bench.py end to end on the GPU at C1's shape (OPT-125m fp32, small enough
to run in seconds): the JSON line the driver reads, for the eager step, the
captured-graph step and plain MeZO, and the kernel microbench.

Each run is a child process (`python bench.py ...`), as the driver runs it.
With 3 timed steps and 1 warm-up step the step counter is placed so that the
DiZO event falls on the last timed step: the event's 42 projection launches
(1 norm, 21 applies, 20 reverse + norm passes over the 24 k/v groups) and the
restore + update before it are spread over 50 steps, so every line reports
2 + 43 / 50 library launches per step."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    cmd = [sys.executable, "bench.py", *args]
    print("running", " ".join(cmd[1:]), flush=True)
    out = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-3000:]
    lines = [ln for ln in out.stdout.splitlines() if ln.startswith("{")]
    assert len(lines) == 1, out.stdout[-2000:]
    return json.loads(lines[0])


@pytest.fixture(scope="module")
def eager():
    return _bench("--workload", "c1", "--steps", "3", "--warmup", "1", "--no-cpu-baseline")


def test_step_line(eager):
    d = eager
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1 and d["dtype"] == "fp32"
    assert d["value"] > 0 and abs(d["ms_per_step"] - 1000.0 / d["value"]) < 1e-9
    assert d["config"]["dizo_events_timed"] == 1
    r = d["roofline"]
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert 0.2 < r["frac"] < 1.0 and abs(r["frac"] - r["achieved"] / r["peak"]) < 1e-12
    assert r["algorithmic_bytes_per_launch"] == 2 * 4 * d["config"]["zo_params"]
    assert abs(r["library_launches_per_step"] - (2 + 43 / 50)) < 1e-12
    assert r["event_amortisation"]["launches_per_event"] == 43
    k = d["kernels"]
    assert k["restore_update_perturb"]["launches"] == 2 and k["perturb"]["launches"] == 4
    assert k["proj_apply"]["launches"] == 21 and k["proj_reverse_sumsq"]["launches"] == 20


def test_graph_step_line_matches_eager(eager):
    """Captured steps: the replays are not timed, so there is no roofline
    kernel time, but the amortised launches and bytes come from the step's
    structure and equal the eager line's, and the losses are the eager ones bit
    for bit."""
    d = _bench("--workload", "c1", "--steps", "3", "--warmup", "1", "--no-cpu-baseline", "--graph")
    assert d["config"]["graph"] is True and d["value"] > 0
    r, re_ = d["roofline"], eager["roofline"]
    assert r["frac"] is None
    assert abs(r["library_launches_per_step"] - re_["library_launches_per_step"]) < 1e-12
    assert abs(r["bytes_per_param_per_step"] - re_["bytes_per_param_per_step"]) < 1e-12
    assert d["loss_first_last"] == eager["loss_first_last"]


def test_mezo_line_has_no_event():
    """Plain MeZO: no event; the window's own launches, 7 in 3 steps (the
    first step's +1, three -2, two fused restore + update + next perturb and
    the restore + update that ends the window)."""
    d = _bench("--workload", "c1", "--steps", "3", "--warmup", "1", "--no-cpu-baseline", "--enhanced", "none")
    r = d["roofline"]
    assert d["config"]["dizo_events_timed"] == 0 and r["event_amortisation"] is None
    assert abs(r["library_launches_per_step"] - 7 / 3) < 1e-12
    assert abs(r["bytes_per_param_per_step"] - 7 * 2 * 4 / 3) < 1e-12


def test_kernel_microbench_line():
    d = _bench("--kernels", "--workload", "c1", "--no-cpu-baseline")
    assert d["metric"] == "ZO pass HBM GB/s" and d["bytes_per_pass"] > 0
    for name in ("perturb+1", "restore_update", "restore_update_perturb", "proj_apply", "proj_reverse_sumsq"):
        p = d["passes"][name]
        assert p["ms"] > 0 and 0.1 < p["frac"] < 1.0, (name, p)
