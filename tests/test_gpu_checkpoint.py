"""ZO journal replay and checkpoint resume on the GPU (dizo_amd.checkpoint).

Replay: a run's journal applied to the weights it started from reproduces
its final weights bit for bit, with no forward, including DiZO events (ZO
and first-order) and captured-graph steps. Resume: a run restored from a
checkpoint written mid-run and continued gives the uninterrupted run's
losses, weights and gamma bit for bit (numpy seed stream, LR schedule,
DiZO state, first-order Adam state, gamma-search loader position)."""
import copy

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().view({2: torch.int16, 4: torch.int32}[t.element_size()])


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(_bits(a), _bits(b))


def _batches():
    from dizo_amd.synth import make_batches
    return make_batches(5, 4, 512, seed=61, device="cuda", min_len=8, max_len=20)


def _trainer(dt, enhanced, graph=False, journal=True, seed=71, fused=False):
    from dizo_amd.synth import Cycle, build_opt
    from dizo_amd.trainer import ZOArguments, ZOTrainer
    model = build_opt("opt-tiny", dt, "cuda", seed=seed)
    init = copy.deepcopy(model)
    args = ZOArguments(learning_rate=1e-3, zo_eps=1e-3, max_steps=120, enhanced=enhanced, zo_graph=graph,
                       zo_journal=journal, zo_fused_mlp=fused, zo_fused_qkv=fused)
    np.random.seed(26)
    tr = ZOTrainer(model, args, train_dataloader=Cycle(_batches()))
    return tr, model, init


def _run(tr, it, n):
    return [tr.training_step(next(it)).reshape(()).clone() for _ in range(n)]


@pytest.mark.parametrize("dt,enhanced,graph", [
    (torch.float16, None, False), (torch.bfloat16, None, False), (torch.float32, None, False),
    (torch.float16, "zo", False), (torch.bfloat16, "zo", False), (torch.float16, "fo", False),
    (torch.float16, "zo", True), (torch.bfloat16, None, True), (torch.float16, "grid", False),
])
def test_replay_reproduces_the_run(dt, enhanced, graph, tmp_path):
    """55 steps (a DiZO event at global step 49 when enhanced): replaying the
    journal, saved and loaded as JSON, onto the initial weights gives the
    run's weights bit for bit; a replay cut after 30 steps gives the weights
    the run had after step 30."""
    from dizo_amd.checkpoint import ZOJournal, replay
    from dizo_amd.synth import Cycle
    tr, model, init = _trainer(dt, enhanced, graph)
    it = iter(Cycle(_batches()))
    _run(tr, it, 30)
    tr.zo_flush()
    mid = [p.detach().clone() for p in model.parameters()]
    _run(tr, it, 25)
    tr.zo_close()
    torch.cuda.synchronize()
    path = str(tmp_path / "journal.json")
    tr.zo_journal.save(path)
    journal = ZOJournal.load(path)
    assert journal.steps == 55
    n_proj = sum(1 for op in journal.ops if op[0] != "zo")
    assert n_proj == {None: 0, "zo": 41, "fo": 1, "grid": 1}[enhanced]

    fresh, anchor = copy.deepcopy(init), copy.deepcopy(init)
    assert replay(fresh, journal, base_model=anchor) == 55
    torch.cuda.synchronize()
    bad = [n for (n, a), b in zip(fresh.named_parameters(), model.parameters()) if not _same(a.data, b.data)]
    assert not bad, f"{len(bad)} tensors differ after replay, e.g. {bad[:3]}"

    part = copy.deepcopy(init)
    assert replay(part, journal, base_model=anchor, upto=30) == 30
    torch.cuda.synchronize()
    assert all(_same(a.data, b) for a, b in zip(part.parameters(), mid))
    if dt == torch.float16 and enhanced is None:
        changed = sum(1 for a, b in zip(init.parameters(), model.parameters()) if not _same(a.data, b.data))
        assert changed > 0


@pytest.mark.parametrize("enhanced,fused", [("zo", False), ("fo", False), ("zo", True), ("fo", True)])
def test_resume_from_checkpoint_is_exact(enhanced, fused, tmp_path):
    """110 steps uninterrupted against 60 steps, a checkpoint, and a fresh
    trainer that loads it and runs the last 50 (DiZO events at global steps 49
    and 99, so the second event depends on restored state). fused: the
    decoder layers in the fused forms, whose k/v/q weights share one storage
    (saved as separate tensors, loaded back in place)."""
    from dizo_amd.checkpoint import load_checkpoint, replay, save_checkpoint
    from dizo_amd.synth import Cycle
    dt = torch.float16
    tr_a, model_a, init = _trainer(dt, enhanced, fused=fused)
    it = iter(Cycle(_batches()))
    _run(tr_a, it, 60)
    save_checkpoint(tr_a, str(tmp_path / "ckpt"))
    tail_a = _run(tr_a, it, 50)
    gamma_a = tr_a.dizo_trainer.dizo.gamma().clone()
    tr_a.zo_close()

    tr_b, model_b, _ = _trainer(dt, enhanced, seed=99, fused=fused)  # different initial weights: all come from the checkpoint
    np.random.seed(1)  # and a different seed stream: it comes from the checkpoint too
    load_checkpoint(tr_b, str(tmp_path / "ckpt"))
    assert tr_b.state.global_step == 60
    it_b = iter(Cycle(_batches()))
    for _ in range(60):
        next(it_b)
    tail_b = _run(tr_b, it_b, 50)
    gamma_b = tr_b.dizo_trainer.dizo.gamma().clone()
    tr_b.zo_close()
    torch.cuda.synchronize()
    assert all(_same(a, b) for a, b in zip(tail_a, tail_b)), "losses after the resume differ"
    assert _same(gamma_a, gamma_b)
    for (n, a), b in zip(model_a.named_parameters(), model_b.parameters()):
        assert _same(a.data, b.data), n
    # the restored journal covers the whole run: replaying it from the initial
    # weights gives the same final weights
    assert tr_b.zo_journal.steps == 110
    fresh = copy.deepcopy(init)
    replay(fresh, tr_b.zo_journal, base_model=copy.deepcopy(init))
    torch.cuda.synchronize()
    named_a = dict(model_a.named_parameters())
    for n, p in fresh.named_parameters():
        assert _same(p.data, named_a[n].data), n
