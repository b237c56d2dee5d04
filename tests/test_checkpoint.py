"""Host logic of the ZO journal / checkpoint format (dizo_amd.checkpoint): the
replay plan, exact JSON round trips, the first-order rollback and the layout
check. No kernels run here; tests/test_gpu_checkpoint.py replays on the GPU."""
import json

import numpy as np
import pytest
import torch

from dizo_amd import checkpoint as C
from dizo_amd._lib import DzError


def _journal():
    return C.ZOJournal([("a.weight", 12, "float16"), ("b.weight", 5, "float16")], 1e-3, ["a.weight"])


def test_replay_plan_fuses_like_the_trainer():
    """Consecutive steps fuse restore+update with the next +1; a projection op
    (or the end) first applies the pending restore+update unfused."""
    a = torch.ones(1, dtype=torch.float16)
    ops = [["zo", 1, 0.5, 1e-6], ["zo", 2, -1.0, 1e-6], ["apply", a], ["reverse", a], ["zo", 3, 2.0, 9e-7],
           ["zo", 4, 0.25, 8e-7]]
    plan = C.replay_plan(ops)
    assert [p[0] for p in plan] == ["perturb", "perturb", "restore_update_perturb", "perturb", "restore_update",
                                    "proj", "proj", "perturb", "perturb", "restore_update_perturb", "perturb",
                                    "restore_update"]
    assert plan[0] == ("perturb", 1, 1.0) and plan[1] == ("perturb", 1, -2.0)
    assert plan[2] == ("restore_update_perturb", (1, 0.5, 1e-6), 2)
    assert plan[4] == ("restore_update", (2, -1.0, 1e-6))
    assert plan[5][1] == "apply" and plan[6][1] == "reverse"
    assert plan[7] == ("perturb", 3, 1.0)
    assert plan[-1] == ("restore_update", (4, 0.25, 8e-7))
    assert C.replay_plan([]) == []


def test_every_step_is_applied_once_by_the_plan():
    """Each zo op contributes exactly +1 (alone or fused), -2 and one restore+update."""
    rng = np.random.default_rng(0)
    for _ in range(50):
        ops = []
        for _ in range(int(rng.integers(0, 12))):
            if rng.random() < 0.7:
                ops.append(["zo", int(rng.integers(1e9)), float(rng.normal()), 1e-6])
            else:
                ops.append(["apply", torch.ones(1)])
        plan = C.replay_plan(ops)
        seeds = [op[1] for op in ops if op[0] == "zo"]
        plus = [p[1] for p in plan if p[0] == "perturb" and p[2] == 1.0] + \
               [p[2] for p in plan if p[0] == "restore_update_perturb"]
        minus = [p[1] for p in plan if p[0] == "perturb" and p[2] == -2.0]
        restored = [p[1][0] for p in plan if p[0] in ("restore_update", "restore_update_perturb")]
        assert sorted(plus) == sorted(seeds) and minus == seeds and restored == seeds
        assert sum(1 for p in plan if p[0] == "proj") == len(ops) - len(seeds)


def test_json_round_trip_is_exact(tmp_path):
    j = _journal()
    j.zo(123456789, 0.7109375, 9.93875e-07)
    j.zo(5, torch.tensor(-3.25, dtype=torch.float16), 1e-6)  # a captured step's device-side g
    vals = [0.9003906, 1.0, 6.1e-05, 2.0 ** -24, 65504.0]
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        j.proj("apply" if dt != torch.float32 else "apply_f32", torch.tensor(vals, dtype=torch.float32).to(dt))
    j.proj("reverse", torch.tensor([0.75], dtype=torch.float16))
    path = str(tmp_path / "journal.json")
    j.save(path)
    k = C.ZOJournal.load(path)
    assert k.layout == j.layout and k.eps == j.eps and k.projected == j.projected and k.steps == 2
    assert k.ops[0] == ["zo", 123456789, 0.7109375, 9.93875e-07]
    assert k.ops[1] == ["zo", 5, -3.25, 1e-6]
    for a, b in zip(j.ops[2:], k.ops[2:]):
        assert a[0] == b[0] and a[1].dtype == b[1].dtype and torch.equal(a[1], b[1])


def test_first_order_iterations_roll_back():
    j = _journal()
    j.zo(1, 0.5, 1e-6)
    for _ in range(3):  # an iteration: snapshot, apply, restore
        j.mark()
        j.proj("apply_f32", torch.ones(1))
        j.rollback()
    j.proj("apply_f32", torch.full((1,), 0.9))  # the final apply stays
    j.rollback()  # no mark: nothing to drop
    assert [op[0] for op in j.ops] == ["zo", "apply_f32"]


def test_format_and_layout_checks():
    with pytest.raises(DzError):
        C.ZOJournal.from_json({"format": "something-else", "version": 1})
    d = _journal().to_json()
    d["ops"] = [["bogus"]]
    with pytest.raises(DzError):
        C.ZOJournal.from_json(d)
    with pytest.raises(DzError):
        _journal().proj("scale", torch.ones(1))
    j = _journal()
    good = [("a.weight", torch.zeros(12, dtype=torch.float16)), ("b.weight", torch.zeros(5, dtype=torch.float16))]
    C._check_layout(j, good)
    with pytest.raises(DzError, match="tensor 1"):
        C._check_layout(j, [good[0], ("b.weight", torch.zeros(6, dtype=torch.float16))])
    with pytest.raises(DzError, match="tensor 0"):
        C._check_layout(j, [("a.weight", torch.zeros(12, dtype=torch.bfloat16)), good[1]])
    with pytest.raises(DzError, match="has 2 tensors"):
        C._check_layout(j, good[:1])


def test_numpy_rng_state_round_trips():
    np.random.seed(26)
    np.random.randint(1000000000)
    s = json.loads(json.dumps(C._np_state()))
    want = [np.random.randint(1000000000) for _ in range(5)]
    np.random.seed(0)
    C._set_np_state(s)
    assert [np.random.randint(1000000000) for _ in range(5)] == want
