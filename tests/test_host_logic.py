"""Host-side behaviour of the drop-in trainer that needs no kernel, on the
CPU: the NaN/inf loss filter (trainer.py:1242-1250), the stop-on-signal
contract (utils.py:291-315 with trainer.py:1357), a checkpoint written and
read back on the CPU, and the per-step JSON log."""
import json
import os
import signal

import numpy as np
import pytest
import torch


@pytest.fixture()
def cpu_trainer(tmp_path):
    from transformers import OPTForCausalLM

    from dizo_amd.synth import SHAPES, opt_config
    from dizo_amd.trainer import ZOArguments, ZOTrainer

    torch.manual_seed(0)
    model = OPTForCausalLM(opt_config(SHAPES["opt-tiny"])).eval()
    args = ZOArguments(learning_rate=1e-6, max_steps=10, zo_log_path=str(tmp_path / "steps.jsonl"))
    np.random.seed(26)
    tr = ZOTrainer(model, args)
    yield tr


def test_nan_inf_filter_matches_reference_loop(cpu_trainer):
    """The device-side filter (torch.where, no sync) against the reference's
    branch, step by step, with NaN and inf losses among finite ones."""
    tr = cpu_trainer
    losses = [0.7, 0.69, float("nan"), 0.71, float("inf"), 0.68, float("-inf"), 0.7, float("nan")]
    ref = torch.tensor(0.0)  # trainer.py:1121
    last_logged = 0           # trainer.py:1124 (never updated by the ZO loop)
    for k, x in enumerate(losses):
        step = torch.tensor(x, dtype=torch.float16)
        if torch.isnan(step) or torch.isinf(step):
            ref += ref / (1 + k - last_logged)
        else:
            ref += step
        tr.state.global_step = k
        tr._account(step)
        assert tr.tr_loss.dtype == torch.float32
        assert torch.equal(tr.tr_loss.view(torch.int32), ref.view(torch.int32)), (k, float(tr.tr_loss), float(ref))


def test_signal_stops_at_the_end_of_the_step(cpu_trainer, tmp_path):
    """SIGUSR1 during step 3 ends the run after that step; the pending work is
    flushed and a checkpoint is written, which a fresh trainer reads back
    (step counter, numpy seed stream, learning rate)."""
    from dizo_amd.checkpoint import load_checkpoint
    from dizo_amd.trainer import StopOnSignal
    tr = cpu_trainer
    calls = []

    def fake_step(inputs):
        calls.append(inputs)
        tr.zo_random_seed = np.random.randint(1000000000)
        tr.state.global_step += 1
        tr.lr_scheduler.step()
        if len(calls) == 3:
            os.kill(os.getpid(), signal.SIGUSR1)
        return torch.tensor(0.5)

    tr.training_step = fake_step
    flushed = []
    tr.zo_flush = lambda: flushed.append(True)
    stop = StopOnSignal()
    try:
        tr.train(range(100), max_steps=10, stop=stop, checkpoint_dir=str(tmp_path / "ckpt"))
    finally:
        stop.close()
    assert len(calls) == 3 and stop.signal_received and flushed
    assert tr.state.global_step == 3
    want_next = np.random.randint(1000000000)

    from transformers import OPTForCausalLM

    from dizo_amd.synth import SHAPES, opt_config
    from dizo_amd.trainer import ZOArguments, ZOTrainer
    torch.manual_seed(1)
    other = ZOTrainer(OPTForCausalLM(opt_config(SHAPES["opt-tiny"])).eval(), ZOArguments(learning_rate=1e-6,
                                                                                         max_steps=10))
    np.random.seed(5)
    load_checkpoint(other, str(tmp_path / "ckpt"))
    assert other.state.global_step == 3
    assert other._get_learning_rate() == tr._get_learning_rate()
    assert np.random.randint(1000000000) == want_next
    for (n, a), (_, b) in zip(tr.model.named_parameters(), other.model.named_parameters()):
        assert torch.equal(a, b), n


def test_step_log_writes_json_lines(cpu_trainer):
    tr = cpu_trainer
    for k in range(3):
        tr.zo_random_seed = 100 + k
        tr._log_step(torch.tensor(0.5 + k), torch.tensor(0.25), 1.5 * k, 1e-6)
        tr.state.global_step += 1
    tr.flush_log()
    lines = [json.loads(x) for x in open(tr._log_path)]
    assert [x["step"] for x in lines] == [1, 2, 3]
    assert [x["seed"] for x in lines] == [100, 101, 102]
    assert lines[2] == {"step": 3, "seed": 102, "loss1": 2.5, "loss2": 0.25, "projected_grad": 3.0, "lr": 1e-6}


def test_train_runs_epochs_over_a_short_batch_list(cpu_trainer):
    """A list shorter than max_steps is run again from its start (one epoch
    after another, as the reference's loop does); a one-shot iterator ends the
    run when it is exhausted; an empty list is an error."""
    from dizo_amd._lib import DzError
    tr = cpu_trainer
    seen = []

    def fake_step(inputs):
        seen.append(inputs)
        tr.state.global_step += 1
        tr.loss_list.append(torch.tensor(0.5))
        return torch.tensor(0.5)

    tr.training_step = fake_step
    tr.zo_flush = lambda: None
    tr.train(["a", "b", "c"], max_steps=7)
    assert seen == ["a", "b", "c", "a", "b", "c", "a"]
    assert tr.state.epoch == 2.0
    seen.clear()
    tr.train(iter(["x", "y"]), max_steps=5)
    assert seen == ["x", "y"]
    with pytest.raises(DzError):
        tr.train([], max_steps=2)
