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
    assert set(bench.WORKLOADS) == {"c1", "c2", "c3", "c4", "c5"}
    assert bench.WORKLOADS["c2"]["kernels_only"] and bench.WORKLOADS["c2"]["shape"] == "opt-2.7b"
    c4 = bench.WORKLOADS["c4"]
    assert (c4["shape"], c4["dtype"], c4["batch"], c4["fixed_len"]) == ("opt-13b", "float16", 16, 128)
    for flags in (["--graph"], ["--full-logits"], ["--hf-layers"], ["--kernels"],
                  ["--enhanced", "fo"],
                  ["--workload", "c5"], ["--workload", "c2", "--kernels"], ["--no-cpu-baseline"]):
        assert bench.main(flags + ["--gpus", "3"]) == 2  # parses, then stops at the one-GPU check


def test_event_lands_in_every_timed_window():
    """The step counter offset puts the DiZO event (after the update of every
    50th step) on timed step min(steps, 50) - 1, whatever the warm-up."""
    for steps in (1, 5, 20, 49, 50, 51, 120):
        for warmup in (0, 1, 3, 5, 49, 50, 77):
            off = bench.event_offset(steps, warmup)
            timed = [off + warmup + j for j in range(steps)]
            events = [j for j, g in enumerate(timed) if (g + 1) % 50 == 0]
            assert events and events[0] == min(steps, 50) - 1, (steps, warmup, off, events)


def test_amortised_rate():
    # 20 steps in 5 s of which one 2 s event: 3 s of steps; one event per 50 steps adds 2 * 20 / 50 = 0.8 s
    v, zo, ev = bench.amortised(20, 5.0, [2.0])
    assert abs(v - 20 / 3.8) < 1e-12 and abs(zo - 20 / 3.0) < 1e-12 and ev == 2.0
    # 50 steps with one event: the plain rate
    v, _, _ = bench.amortised(50, 10.0, [2.0])
    assert abs(v - 5.0) < 1e-12
    assert bench.amortised(10, 2.0, []) == (5.0, 5.0, None)


def test_amortised_passes_spread_the_event_over_fifty_steps():
    # the window of a 20-step run with the event on its last step (C4 fp16):
    # 20 x -2, 19 three-way, 1 restore+update before the event, 1 +1 after it;
    # the event's 1 sumsq, 21 apply and 20 reverse+norm passes
    P, b, kv = 12_596_080_640, 50_384_322_560.0, 2_097_152_000
    summ = {"perturb": {"launches": 21, "bytes_per_launch": b},
            "restore_update_perturb": {"launches": 19, "bytes_per_launch": b},
            "restore_update": {"launches": 1, "bytes_per_launch": b},
            "proj_sumsq": {"launches": 1, "bytes_per_launch": 4.0 * kv},
            "proj_apply": {"launches": 21, "bytes_per_launch": 6.0 * kv},
            "proj_reverse_sumsq": {"launches": 20, "bytes_per_launch": 6.0 * kv}}
    got = bench.amortised_passes(summ, 20, 1, P, b)
    # per 50 steps: 101 RMW launches (2 per step and 1 around the event) and 42 projection launches
    assert abs(got["library_launches_per_step"] - (101 + 42) / 50) < 1e-12
    want = (101 * b + (4 + 41 * 6) * kv) / 50 / P
    assert abs(got["bytes_per_param_per_step"] - want) < 1e-12
    # the same window read over more steps gives the same amortised figures
    summ2 = dict(summ, perturb={"launches": 51, "bytes_per_launch": b},
                 restore_update_perturb={"launches": 49, "bytes_per_launch": b})
    got2 = bench.amortised_passes(summ2, 50, 1, P, b)
    assert abs(got2["library_launches_per_step"] - got["library_launches_per_step"]) < 1e-12
    # without events: the window's own figures
    none = bench.amortised_passes({"perturb": {"launches": 10, "bytes_per_launch": b}}, 5, 0, P, b)
    assert none["library_launches_per_step"] == 2 and none["event_amortisation"] is None
    # captured-graph replays: only the event's passes are timed; the ZO launches come from the
    # step's structure (2 per step, 1 more per event) and give the eager figures
    graph = {k: v for k, v in summ.items() if k.startswith("proj_")}
    got3 = bench.amortised_passes(graph, 20, 1, P, b)
    assert abs(got3["library_launches_per_step"] - got["library_launches_per_step"]) < 1e-12
    assert abs(got3["bytes_per_param_per_step"] - got["bytes_per_param_per_step"]) < 1e-12
