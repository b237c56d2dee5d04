"""CPU checks of bench.py's command-line contract (no GPU is touched).

The driver runs `python bench.py --gpus N --steps K --warmup W` and reads one
JSON line from stdout. This build measures one GPU: N > 1 must exit non-zero
with a JSON line that says so, before anything initialises a device; with no
GPU visible the line reports that instead of a number.
"""
import json

import pytest

import bench


def _last_json(out: str) -> dict:
    lines = [ln for ln in out.strip().splitlines() if ln.startswith("{")]
    assert lines, out
    return json.loads(lines[-1])


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_exits_with_a_message(n, capsys):
    rc = bench.main(["--gpus", str(n), "--steps", "5", "--warmup", "1"])
    line = _last_json(capsys.readouterr().out)
    assert rc == 2 and line["n_gpus"] == n and "one GPU" in line["error"]


def test_no_gpu_reports_an_error_line(capsys):
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    rc = bench.main(["--steps", "1", "--warmup", "0"])
    assert rc == 1 and "error" in _last_json(capsys.readouterr().out)


def test_flags_and_workloads():
    assert set(bench.WORKLOADS) == {"c1", "c3", "c4", "c5"}
    c4 = bench.WORKLOADS["c4"]
    assert (c4["shape"], c4["dtype"], c4["batch"], c4["fixed_len"]) == ("opt-13b", "float16", 16, 128)
    for flags in (["--graph"], ["--full-logits"], ["--hf-layers"], ["--sdpa"], ["--dz-attention"], ["--kernels"],
                  ["--enhanced", "fo"],
                  ["--workload", "c5"], ["--no-cpu-baseline"]):
        assert bench.main(flags + ["--gpus", "3"]) == 2  # parses, then stops at the one-GPU check
