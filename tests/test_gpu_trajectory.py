"""Long-run parity of the drop-in trainer against the reference's expressions,
and the per-pass contract at OPT-2.7B tensor shapes.

The reference side runs the reference's torch expressions (oracle.ref_torch:
trainer.py:1429-1444, 1570-1617, 405-465, 545-614) on ROCm torch, fed the z
and gamma noise the library exports, with the same numpy seed stream, batches
and learning-rate schedule:

  * 200 steps with a DiZO event every 50 (ENHANCED=zo), on a small model:
    with the library's norm definition on the reference side (fp64 sum of
    squares, correctly rounded), losses, gamma and every weight agree bit for
    bit at fp16 / bf16 / fp32;
  * the same 200 steps at config C3's shape (OPT-2.7B fp16, batch 16 x 2
    candidates, lengths uniform in [32, 64]): bit for bit against the
    reference's expressions rounded as torch's CPU and CUDA kernels round
    them, with that norm; against ROCm torch's own kernels and torch.norm,
    within 1e-2, and where that run leaves the recipe (fp32 ties that ROCm
    torch rounds the other way) asserted element by element;
  * config C2 (kernel passes over the OPT-2.7B trainable set): separate
    passes (+1, -2, +1, update) and fused passes give the same weights bit for
    bit, and match the reference's expressions on sampled tensors;
  * config C5's scale (OPT-30B bf16) and config C4, the headline (OPT-13B
    fp16): the fused passes and the projection on sampled tensors and groups
    against the reference's expressions; whole steps, forwards included, bit
    for bit: at C4 three, and fifty ending in a DiZO event; at C5 two.

Both sides run the model's forward on PyTorch (hipBLASLt GEMMs, SDPA). That
forward is not bitwise repeatable in rare cases on this stack: with the
weights and the batch fixed and only torch work between them, 1 of 2400 C4
forwards gave a loss one unit in the last place away (a run with no library
kernel in the loop). The bit-for-bit runs therefore compare each step
forward's loss with the library's (_Agreement): a reference forward that
differs is recomputed once, the run continues from the library's value, and
the step is noted; at most one note is allowed, and every weight, gamma and
the other losses must still agree bit for bit. The SPSA forwards of the DiZO
events are compared the same way. The captured-graph test, which compares two
whole runs, counts a difference only if it survives one more run of each form.
"""
import copy
import sys

import numpy as np
import pytest
import torch

from oracle import arith as A
from oracle import ref_torch as R

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().view({2: torch.int16, 4: torch.int32}[t.element_size()])


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(_bits(a), _bits(b))


def _lib_norm(t: torch.Tensor) -> torch.Tensor:
    s = (t.double() ** 2).sum().float()
    return torch.sqrt(s.double()).float().to(t.dtype)


def _reporter(capsys):
    """A progress callback that prints every 50 steps with pytest's output
    capture suspended, so a long run shows that it is moving."""
    def report(what: str, k: int, steps: int) -> None:
        if (k + 1) % 50 == 0 or k + 1 == steps:
            with capsys.disabled():
                sys.stdout.write(f"  [{what}] step {k + 1}/{steps}\n")
                sys.stdout.flush()
    return report


def _quiet(what: str, k: int, steps: int) -> None:
    pass


def _ref_forward(model, batch):
    from dizo_amd.trainer import forward_wrap_with_option_len
    model.eval()
    with torch.inference_mode():
        return forward_wrap_with_option_len(model, **batch, return_dict=True).loss.detach()


def _library_run(shape, dt, batches, steps, lr0, eps, seed=5, progress=_quiet, **zo_args):
    """The library trainer (ENHANCED=zo, fused passes; zo_args: further
    ZOArguments). Returns the trainer (kept open for export_z), its losses, its
    model and a copy of the initial model."""
    from dizo_amd.synth import Cycle, build_opt
    from dizo_amd.trainer import ZOArguments, ZOTrainer
    model = build_opt(shape, dt, "cuda", seed=seed)
    init = copy.deepcopy(model)
    args = ZOArguments(learning_rate=lr0, zo_eps=eps, max_steps=steps, enhanced="zo", **zo_args)
    np.random.seed(26)
    tr = ZOTrainer(model, args, train_dataloader=Cycle(batches))
    if args.enhanced == "zo":
        _trace_events(tr)
    losses, losses2 = [], []
    for k in range(steps):
        losses.append(tr.training_step(batches[k % len(batches)]).reshape(()).clone())
        l2 = getattr(tr, "_last_loss2", None)
        losses2.append(l2.reshape(()).clone() if l2 is not None else None)
        progress(f"library {shape}", k, steps)
    tr.zo_flush()
    torch.cuda.synchronize()
    tr.test_step_losses = (losses, losses2)
    return tr, losses, model, init


def _trace_events(tr) -> None:
    """Records the two losses of every SPSA iteration of the library's DiZO
    events (DiZO.zo_forward keeps the last pair) in tr.test_event_losses."""
    dz = tr.dizo_trainer.dizo
    inner = dz.zo_forward
    tr.test_event_losses = []

    def traced(*a, **k):
        out = inner(*a, **k)
        if not k.get("apply", False):
            tr.test_event_losses.append(tuple(x.reshape(()).clone() for x in dz.last_losses))
        return out

    dz.zo_forward = traced


class _Agreement:
    """The library run's forward losses (L1 and L2 of every step, and of every
    SPSA iteration of its events), which the reference run's forwards are
    compared with (module doc)."""

    def __init__(self, tr, limit: int = 1):
        self.lib = tr.test_step_losses
        self.ev = getattr(tr, "test_event_losses", [])
        self.limit = limit
        self.notes = []

    def _agree(self, value, want, what, recompute):
        if _same(value.reshape(()), want):
            return value
        again = recompute()
        self.notes.append((what, float(value), float(again), float(want)))
        return want.reshape(value.shape).clone()

    def agree(self, value, which: int, k: int, recompute):
        """Step k's forward `which` (0: L1, 1: L2)."""
        return self._agree(value, self.lib[which][k], f"step {k} L{which + 1}", recompute)

    def agree_event(self, value, n: int, j: int, recompute):
        """Forward j of SPSA iteration n (counted over the run's events)."""
        return self._agree(value, self.ev[n][j], f"SPSA iteration {n} forward {j + 1}", recompute)

    def check(self) -> None:
        for what, first, again, lib in self.notes:
            print(f"{what}: reference forward {first}, recomputed {again}; library {lib}")
        assert len(self.notes) <= self.limit, f"{len(self.notes)} forwards disagree: {self.notes[:4]}"


def _reference_run(tr, init, dt, batches, steps, lr0, eps, norm, recipe=False, progress=_quiet, ops=None,
                   agree=None):
    """The reference's expressions on a copy of the initial model, fed the z and
    gamma noise the library exports. recipe: the perturbation and update
    evaluated in the recipe form (exact products rounded as torch's CPU and
    CUDA kernels round them) instead of by ROCm torch's fused kernels. ops: an
    object with perturb / update methods of the same signatures, used instead
    of either form (given the step index through ops.step; the run ends before
    a step once ops.stop is set). agree: an _Agreement with the library run's
    step losses, for the runs expected to match it bit for bit.
    Returns (losses, model, gamma)."""
    from dizo_amd import _lib as L
    from dizo_amd.synth import Cycle
    from dizo_amd.table import normals
    from dizo_amd.trainer import select_trainable
    model_b, anchor_b = copy.deepcopy(init), copy.deepcopy(init)
    np.random.seed(26)
    named_b, _ = select_trainable(model_b)
    names = [n for n, _ in named_b]
    params_b = [p for _, p in named_b]
    proj = tr.dizo_trainer.dizo.constraints_name
    G = len(proj)
    pgm = iter(Cycle(batches))
    dev = torch.device("cuda", 0)
    losses, gammas = [], None
    for k in range(steps):
        if ops is not None and ops.stop:
            break
        seed = np.random.randint(1000000000)
        zs = [tr.export_z(n, seed) for n in names]
        batch = batches[k % len(batches)]
        perturb = R.zo_perturb_parameters_recipe if recipe else R.zo_perturb_parameters
        update = R.zo_update_recipe if recipe else R.zo_update
        if ops is not None:
            ops.step = k
            perturb, update = ops.perturb, ops.update
        perturb(params_b, zs, 1, eps)
        l1 = _ref_forward(model_b, batch)
        if agree is not None:
            l1 = agree.agree(l1, 0, k, lambda: _ref_forward(model_b, batch))
        perturb(params_b, zs, -2, eps)
        l2 = _ref_forward(model_b, batch)
        if agree is not None:
            l2 = agree.agree(l2, 1, k, lambda: _ref_forward(model_b, batch))
        g = R.projected_grad(l1, l2, eps)
        perturb(params_b, zs, 1, eps)
        update(params_b, zs, g, A.zo_lr(lr0, k, steps))
        del zs
        losses.append(l1)
        progress("reference" + (" recipe" if recipe else ""), k, steps)
        if (k + 1) % 50 == 0:
            pb = dict(model_b.named_parameters())
            p0 = dict(anchor_b.named_parameters())
            news, anchors = [pb[n] for n in proj], [p0[n] for n in proj]
            gammas = [torch.nn.Parameter(torch.Tensor([0]).cuda()) for _ in range(G)]
            for it in range(10):
                zg = normals(seed, L.DZ_STREAM_GAMMA, it * G, G, dt, dev)
                data = next(pgm)
                n_it = ((k + 1) // 50 - 1) * 10 + it

                def loss_fn(j, data=data, n_it=n_it):
                    v = _ref_forward(model_b, data)
                    if agree is None:
                        return v
                    return agree.agree_event(v, n_it, j, lambda: _ref_forward(model_b, data))

                R.dizo_zo_iteration(news, anchors, gammas, it == 0, [zg[i:i + 1] for i in range(G)],
                                    loss_fn, norm=norm)
            R.apply_constraints(news, anchors, gammas, norm=norm)
    torch.cuda.synchronize()
    gamma = torch.cat([g.detach().reshape(1) for g in gammas]) if gammas is not None else None
    return losses, model_b, gamma


def _assert_bit_exact(tr, la, ma, lb, mb, gb, agreement=None):
    if agreement is not None:
        agreement.check()
    bad = [k for k, (a, b) in enumerate(zip(la, lb)) if not _same(a, b)]
    assert not bad, f"losses differ at steps {bad[:5]}: {[(float(la[k]), float(lb[k])) for k in bad[:5]]}"
    ga = tr.dizo_trainer.dizo.gamma()
    assert _same(ga, gb), f"gamma {ga} vs {gb}"
    pb = dict(mb.named_parameters())
    diff = [n for n, p in ma.named_parameters() if not _same(p.data, pb[n].data)]
    assert not diff, f"{len(diff)} tensors differ after the run, e.g. {diff[:3]}"


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_200_steps_with_four_dizo_events_bit_exact(dt):
    from dizo_amd.synth import make_batches
    batches = make_batches(7, 4, 512, seed=81, device="cuda", min_len=8, max_len=20)
    tr, la, ma, init = _library_run("opt-tiny", dt, batches, 200, 1e-3, 1e-3)
    ag = _Agreement(tr)
    lb, mb, gb = _reference_run(tr, init, dt, batches, 200, 1e-3, 1e-3, _lib_norm, agree=ag)
    _assert_bit_exact(tr, la, ma, lb, mb, gb, ag)
    tr.zo_close()


def test_c3_shape_200_step_loss_trajectory(capsys):
    """Config C3's shape (OPT-2.7B fp16, batch 16 x 2, lengths U[32, 64], lr 1e-6,
    DiZO events at global steps 49/99/149/199).

    Against the reference's expressions rounded as torch's CPU and CUDA kernels
    round them (the recipe form) and the norm evaluated the library's way, the
    200 steps agree bit for bit: losses, gamma and every weight (north_star's
    1e-3 with no slack).

    Against the recipe form with the reference's own torch.norm (fp32
    accumulation) for the norms, the 200 losses are bit-identical too: the
    norm's accumulation order does not move this run. Asserted within
    north_star's 1e-3.

    Against ROCm torch's own kernels with torch.norm, the runs separate by a few
    fp16 units of the loss: on some launch paths ROCm torch's fp16
    `scalar * tensor` kernel rounds exact fp32 ties away from the recipe (20
    elements of 2,560-element tensors in lr * (g * z) at step 35 here,
    test_c3_rocm_torch_departs_from_the_recipe_only_on_fp32_ties). The ZO
    gradient's fp16 quantisation (steps of 0.25 at eps 1e-3) and the gamma
    search's (L1 - L2) / 0.2 then carry a one-unit weight difference into
    different updates. That run is reported and bounded at 1e-2."""
    from dizo_amd.synth import make_batches
    batches = make_batches(8, 16, 50272, seed=82, device="cuda", min_len=32, max_len=64)
    report = _reporter(capsys)
    tr, la, ma, init = _library_run("opt-2.7b", torch.float16, batches, 200, 1e-6, 1e-3, progress=report)
    ag = _Agreement(tr)
    lb, mb, gb = _reference_run(tr, init, torch.float16, batches, 200, 1e-6, 1e-3, _lib_norm, recipe=True,
                                progress=report, agree=ag)
    _assert_bit_exact(tr, la, ma, lb, mb, gb, ag)
    del mb
    lt, mt, gt = _reference_run(tr, init, torch.float16, batches, 200, 1e-6, 1e-3, torch.norm, progress=report)
    a = torch.stack(la).double().cpu()
    t = torch.stack(lt).double().cpu()
    worst = float((a - t).abs().max())
    same = int((_bits(torch.stack(la)) == _bits(torch.stack(lt))).sum())
    ga = tr.dizo_trainer.dizo.gamma()
    print(f"C3 vs ROCm torch + torch.norm: {same}/200 losses bit-identical, max |dL| = {worst:.3g}, "
          f"gamma max rel diff {float(((ga.double() - gt.double()).abs() / gt.double().abs()).max()):.3g}")
    assert worst <= 1e-2, f"max loss difference {worst} over 200 steps"
    del mt
    # the recipe form with torch.norm: what torch.norm's fp32 accumulation alone changes
    lc, mc, gc = _reference_run(tr, init, torch.float16, batches, 200, 1e-6, 1e-3, torch.norm, recipe=True,
                                progress=report)
    c = torch.stack(lc).double().cpu()
    worst_c = float((a - c).abs().max())
    same_c = int((_bits(torch.stack(la)) == _bits(torch.stack(lc))).sum())
    print(f"C3 vs recipe + torch.norm: {same_c}/200 losses bit-identical, max |dL| = {worst_c:.3g}", flush=True)
    assert worst_c <= 1e-3, f"max loss difference {worst_c} over 200 steps"
    tr.zo_close()


class _TieAudit:
    """The recipe form of trainer.py:1438-1442 and 1603-1608 (what the library
    computes), which at each of the reference's elementwise operations also
    runs ROCm torch's own kernel on the same inputs and records where the two
    differ. For every differing element it checks that the operation's fp32
    result (the exact float64 value rounded to fp32, as torch's CPU and CUDA
    kernels compute it) lies exactly halfway between the recipe's value and
    ROCm torch's, i.e. that the two differ only in how an fp32 tie is rounded
    to the parameter dtype."""

    def __init__(self, names):
        self.names = names
        self.step = -1
        self.stop = False      # set once a step has departed: the runs separate there
        self.departures = []   # (step, op, tensor, numel, count)
        self.non_ties = 0

    def _check(self, rocm, exact64, op, i):
        rec = exact64.float().to(rocm.dtype)
        d = _bits(rec) != _bits(rocm)
        n = int(d.sum())
        if n:
            x = exact64[d].float().double()
            mid = (rec[d].double() + rocm[d].double()) * 0.5
            self.non_ties += int((mid != x).sum())
            self.departures.append((self.step, op, self.names[i], rocm.numel(), n))
            self.stop = True
        return rec

    def perturb(self, params, zs, scaling_factor, zo_eps):
        s, eps = R._f32(scaling_factor), R._f32(zo_eps)
        assert scaling_factor in (1, -2)
        for i, (param, z) in enumerate(zip(params, zs)):
            a = scaling_factor * z   # exact: a product with 1 or -2 is never rounded
            b = self._check(a * zo_eps, a.double() * eps, "(s*z)*eps", i)
            param.data = self._check(param.data + b, param.data.double() + b.double(), "p+b", i)

    def update(self, params, zs, projected_grad, lr):
        g, lr32 = R._f32(projected_grad), R._f32(lr)
        for i, (param, z) in enumerate(zip(params, zs)):
            c = self._check(projected_grad * z, z.double() * g, "g*z", i)
            d = self._check(lr * c, c.double() * lr32, "lr*(g*z)", i)
            param.data = self._check(param.data - d, param.data.double() - d.double(), "p-d", i)


def test_c3_rocm_torch_departs_from_the_recipe_only_on_fp32_ties(capsys):
    """Why ROCm torch's own kernels separate from the library at C3's shape.

    Along the library's 200-step C3 trajectory (the recipe form, bit-exact with
    the library by test_c3_shape_200_step_loss_trajectory), every elementwise
    operation of the reference's perturbation and update is also run by ROCm
    torch's kernel on the same tensors, up to the end of the first step where
    the two differ. Before that step the ROCm torch run is the same run, so its
    differing elements are where that run leaves the recipe. At every one of
    them the fp32 result of the operation is exactly halfway between the two
    values: ROCm torch rounded an fp32 tie to the other neighbour (it rounds
    the exact product once on its non-vectorised launch paths, asserted on
    constructed ties in tests/test_gpu_zo.py)."""
    from dizo_amd.synth import make_batches
    from dizo_amd.trainer import select_trainable
    batches = make_batches(8, 16, 50272, seed=82, device="cuda", min_len=32, max_len=64)
    report = _reporter(capsys)
    tr, la, ma, init = _library_run("opt-2.7b", torch.float16, batches, 200, 1e-6, 1e-3, progress=report)
    del ma
    torch.cuda.empty_cache()
    audit = _TieAudit([n for n, _ in select_trainable(init)[0]])
    ag = _Agreement(tr)
    lb, mb, gb = _reference_run(tr, init, torch.float16, batches, 200, 1e-6, 1e-3, _lib_norm, ops=audit,
                                progress=report, agree=ag)
    ag.check()
    bad = [k for k, (a, b) in enumerate(zip(la, lb)) if not _same(a, b)]
    assert not bad, f"the audited recipe left the library's trajectory at steps {bad[:5]}"
    deps = audit.departures
    assert deps, "ROCm torch's kernels matched the recipe at every operation of the 200 steps"
    total = sum(d[4] for d in deps)
    print(f"ROCm torch vs recipe at C3: first departure at step {deps[0][0]} ({len(lb)} steps audited): "
          f"{total} elements in {len(deps)} tensor ops differ, {audit.non_ties} of them not fp32 ties",
          flush=True)
    for d in deps[:8]:
        print(f"  step {d[0]} {d[1]} {d[2]} ({d[3]} elements): {d[4]}", flush=True)
    assert audit.non_ties == 0
    tr.zo_close()


def test_c4_three_whole_steps_bit_exact():
    """Config C4, the headline (OPT-13B fp16, 643 tensors, batch 16 x 2 x 128,
    unpadded): three whole ZO steps of the library trainer, forwards included,
    against the reference's expressions in the recipe form fed the exported z
    (trainer.py:1570-1608): the losses and every weight bit for bit."""
    from dizo_amd.synth import make_batches
    batches = make_batches(3, 16, 50272, seed=7, device="cuda", fixed_len=128)
    tr, la, ma, init = _library_run("opt-13b", torch.float16, batches, 3, 1e-6, 1e-3)
    assert len(tr.named_parameters_to_optim) == 643
    ag = _Agreement(tr)
    lb, mb, _ = _reference_run(tr, init, torch.float16, batches, 3, 1e-6, 1e-3, _lib_norm, recipe=True, agree=ag)
    print("C4 losses:", [float(x) for x in la], flush=True)
    ag.check()
    bad = [k for k, (a, b) in enumerate(zip(la, lb)) if not _same(a, b)]
    assert not bad, f"losses differ at steps {bad}: {[(float(la[k]), float(lb[k])) for k in bad]}"
    pb = dict(mb.named_parameters())
    diff = [n for n, p in ma.named_parameters() if not _same(p.data, pb[n].data)]
    assert not diff, f"{len(diff)} tensors differ after 3 steps, e.g. {diff[:3]}"
    tr.zo_close()


def test_c4_fifty_steps_with_a_dizo_event_bit_exact(capsys):
    """Config C4 over 50 steps, the last one ending in a DiZO event (10 SPSA
    iterations on the 80 k/v gammas, 20 forwards, the final apply;
    trainer.py:1611-1615, 782-803): the library trainer against the
    reference's expressions in the recipe form with the library's norm
    definition, fed the exported z and gamma noise: losses, gamma and every
    weight bit for bit."""
    from dizo_amd.synth import make_batches
    batches = make_batches(4, 16, 50272, seed=11, device="cuda", fixed_len=128)
    report = _reporter(capsys)
    tr, la, ma, init = _library_run("opt-13b", torch.float16, batches, 50, 1e-6, 1e-3, progress=report)
    ag = _Agreement(tr)
    lb, mb, gb = _reference_run(tr, init, torch.float16, batches, 50, 1e-6, 1e-3, _lib_norm, recipe=True,
                                progress=report, agree=ag)
    _assert_bit_exact(tr, la, ma, lb, mb, gb, ag)
    tr.zo_close()


def test_c5_two_whole_steps_bit_exact():
    """Config C5 (OPT-30B bf16, 771 tensors, 29.6 G elements, batch 8 x 2 x
    256, unpadded): two whole ZO steps of the library trainer, forwards
    included (its three-way pass on the prefetching tile loop), against the
    reference's expressions in the recipe form fed the exported z, one tensor
    at a time (three 59 GB copies of the model fit; a fourth would not): the
    losses and every weight bit for bit."""
    from dizo_amd.synth import make_batches
    from dizo_amd.trainer import select_trainable
    dt, steps, lr0, eps = torch.bfloat16, 2, 1e-6, 1e-3
    batches = make_batches(steps, 8, 50272, seed=13, device="cuda", fixed_len=256)
    tr, la, ma, init = _library_run("opt-30b", dt, batches, steps, lr0, eps)
    named, _ = select_trainable(init)
    assert len(named) == 771
    names = [n for n, _ in named]
    params = [p for _, p in named]  # the copy of the initial model becomes the reference side
    np.random.seed(26)

    def each(op, seed, *args):
        for n, p in zip(names, params):
            z = tr.export_z(n, seed)
            op([p], [z], *args)
            del z

    ag = _Agreement(tr)
    lb = []
    for k in range(steps):
        seed = np.random.randint(1000000000)
        batch = batches[k]
        each(R.zo_perturb_parameters_recipe, seed, 1, eps)
        l1 = ag.agree(_ref_forward(init, batch), 0, k, lambda: _ref_forward(init, batch))
        each(R.zo_perturb_parameters_recipe, seed, -2, eps)
        l2 = ag.agree(_ref_forward(init, batch), 1, k, lambda: _ref_forward(init, batch))
        g = R.projected_grad(l1, l2, eps)
        each(R.zo_perturb_parameters_recipe, seed, 1, eps)
        each(R.zo_update_recipe, seed, g, A.zo_lr(lr0, k, steps))
        lb.append(l1)
    torch.cuda.synchronize()
    print("C5 losses:", [float(x) for x in la], flush=True)
    ag.check()
    bad = [k for k, (a, b) in enumerate(zip(la, lb)) if not _same(a, b)]
    assert not bad, f"losses differ at steps {bad}: {[(float(la[k]), float(lb[k])) for k in bad]}"
    pb = dict(init.named_parameters())
    diff = [n for n, p in ma.named_parameters() if not _same(p.data, pb[n].data)]
    assert not diff, f"{len(diff)} tensors differ after {steps} steps, e.g. {diff[:3]}"
    tr.zo_close()


def test_c5_dizo_event_bit_exact(capsys):
    """Config C5 (OPT-30B bf16, 771 tensors, batch 8 x 2 x 256) with its DiZO
    event: the library trainer started at global step 48, so the event
    (trainer.py:1611-1615, 782-803: 10 SPSA iterations on the 96 k/v gammas
    with 20 forwards, then the final apply) follows the update of the second
    step; against the reference's expressions in the recipe form fed the
    exported z one tensor at a time, the exported gamma noise and the
    library's norm definition: the two losses, the 96 gammas and all 771
    tensors bit for bit."""
    from dizo_amd import _lib as L
    from dizo_amd.synth import Cycle, build_opt, make_batches
    from dizo_amd.table import normals
    from dizo_amd.trainer import ZOArguments, ZOTrainer, select_trainable
    report = _reporter(capsys)
    dt, lr0, eps, steps = torch.bfloat16, 1e-6, 1e-3, 2
    batches = make_batches(3, 8, 50272, seed=17, device="cuda", fixed_len=256)
    model = build_opt("opt-30b", dt, "cuda", seed=0)
    init = copy.deepcopy(model)  # becomes the reference side
    args = ZOArguments(learning_rate=lr0, zo_eps=eps, max_steps=100, enhanced="zo")
    np.random.seed(26)
    tr = ZOTrainer(model, args, train_dataloader=Cycle(batches))
    tr.state.global_step = 48  # the event follows the update of global step 49
    _trace_events(tr)
    proj = tr.dizo_trainer.dizo.constraints_name
    G = len(proj)
    assert G == 96
    p_init = dict(init.named_parameters())
    anchors = [p_init[n].detach().clone() for n in proj]  # theta0 of the projected tensors
    la, la2, lrs = [], [], []
    for k in range(steps):
        lrs.append(float(tr._get_learning_rate()))
        la.append(tr.training_step(batches[k]).reshape(()).clone())
        la2.append(tr._last_loss2.reshape(()).clone())
        report("library c5", k, steps)
    tr.test_step_losses = (la, la2)
    tr.zo_flush()
    torch.cuda.synchronize()
    assert tr.dizo_trainer.i == 1, "the DiZO event did not run"
    g_lib = tr.dizo_trainer.dizo.gamma().detach().clone()

    named, _ = select_trainable(init)
    assert len(named) == 771
    names = [n for n, _ in named]
    params = [p for _, p in named]
    np.random.seed(26)

    def each(op, seed, *a):
        for n, p in zip(names, params):
            z = tr.export_z(n, seed)
            op([p], [z], *a)
            del z

    ag = _Agreement(tr)
    lb = []
    for k in range(steps):
        seed = np.random.randint(1000000000)
        batch = batches[k]
        each(R.zo_perturb_parameters_recipe, seed, 1, eps)
        l1 = ag.agree(_ref_forward(init, batch), 0, k, lambda: _ref_forward(init, batch))
        each(R.zo_perturb_parameters_recipe, seed, -2, eps)
        l2 = ag.agree(_ref_forward(init, batch), 1, k, lambda: _ref_forward(init, batch))
        g = R.projected_grad(l1, l2, eps)
        each(R.zo_perturb_parameters_recipe, seed, 1, eps)
        each(R.zo_update_recipe, seed, g, lrs[k])
        lb.append(l1)
        report("reference c5", k, steps)
    # the event after the second step's update, with that step's seed for the gamma noise
    news = [p_init[n] for n in proj]
    gammas = [torch.nn.Parameter(torch.Tensor([0]).cuda()) for _ in range(G)]
    pgm = iter(Cycle(batches))
    dev = torch.device("cuda", 0)
    for it in range(10):
        zg = normals(seed, L.DZ_STREAM_GAMMA, it * G, G, dt, dev)
        data = next(pgm)

        def loss_fn(j, data=data, it=it):
            return ag.agree_event(_ref_forward(init, data), it, j, lambda: _ref_forward(init, data))

        R.dizo_zo_iteration(news, anchors, gammas, it == 0, [zg[i:i + 1] for i in range(G)], loss_fn,
                            norm=_lib_norm)
        report("reference c5 event", it, 10)
    R.apply_constraints(news, anchors, gammas, norm=_lib_norm)
    torch.cuda.synchronize()
    g_ref = torch.cat([g.detach().reshape(1) for g in gammas])
    print("C5 losses:", [float(x) for x in la], flush=True)
    ag.check()
    bad = [k for k, (a, b) in enumerate(zip(la, lb)) if not _same(a, b)]
    assert not bad, f"losses differ at steps {bad}: {[(float(la[k]), float(lb[k])) for k in bad]}"
    assert _same(g_lib.to(g_ref.dtype), g_ref), f"gamma: {int((_bits(g_lib) != _bits(g_ref)).sum())} of {G} differ"
    pm = dict(model.named_parameters())
    diff = [n for n in names if not _same(pm[n].data, p_init[n].data)]
    assert not diff, f"{len(diff)} tensors differ after the event, e.g. {diff[:3]}"
    tr.zo_close()


def test_c3_shape_fused_forward_bit_identical():
    """The bench's forward at C3's shape (OPT-2.7B fp16, padded batches of 16 x 2
    candidates): with the fused decoder-layer GEMMs, 50 steps with a DiZO event
    give the losses, gamma and weights of HF's layer code bit for bit."""
    from dizo_amd.synth import make_batches

    batches = make_batches(8, 16, 50272, seed=3, device="cuda", min_len=32, max_len=64)
    runs = []
    for fused in (True, False):
        tr, la, ma, _ = _library_run("opt-2.7b", torch.float16, batches, 50, 1e-6, 1e-3, zo_fused_mlp=fused,
                                     zo_fused_qkv=fused, zo_option_head=True)
        runs.append((tr.dizo_trainer.dizo.gamma(), la, {n: p.detach().clone() for n, p in ma.named_parameters()}))
        tr.zo_close()
        del tr, ma
        torch.cuda.empty_cache()
    (ga, la, pa), (gb, lb, pb) = runs
    bad = [k for k, (a, b) in enumerate(zip(la, lb)) if not _same(a, b)]
    assert not bad, f"losses differ at steps {bad[:5]}"
    assert _same(ga, gb)
    diff = [n for n in pa if not _same(pa[n], pb[n])]
    assert not diff, f"{len(diff)} tensors differ, e.g. {diff[:3]}"


def test_c2_opt27b_separate_and_fused_passes():
    """Config C2: perturb +eps, perturb -2 eps, restore +eps and update (g drawn
    N(0,1), lr 1e-6) over the OPT-2.7B trainable set, as separate passes and as
    the fused restore+update and restore+update+next perturb: identical weights;
    the reference's expressions on sampled tensors agree bit for bit."""
    from dizo_amd.synth import build_opt
    from dizo_amd.trainer import _ZOTables, select_trainable
    dt, eps, lr = torch.float16, 1e-3, 1e-6
    g = float(torch.tensor(float(np.random.default_rng(0).standard_normal()), dtype=dt))
    model = build_opt("opt-2.7b", dt, "cuda", seed=0)
    named, _ = select_trainable(model)
    assert len(named) == 515
    sample = [0, len(named) // 2, len(named) - 4]
    before = [named[i][1].detach().clone() for i in sample]
    other = [p.detach().clone() for _, p in named]
    tabs = _ZOTables(named)
    (tab, _), = tabs.tables
    s1, s2 = 1234, 5678
    tab.perturb(s1, 1.0, eps)
    tab.perturb(s1, -2.0, eps)
    tab.perturb(s1, 1.0, eps)
    tab.update(s1, g, lr)
    tab.perturb(s2, 1.0, eps)
    zs = {i: tab.export_z(s1, i) for i in sample}
    torch.cuda.synchronize()
    sep = [p.detach().clone() for _, p in named]
    # reference expressions on the sampled tensors
    for j, i in enumerate(sample):
        ref = [before[j].clone()]
        R.zo_perturb_parameters(ref, [zs[i]], 1, eps)
        R.zo_perturb_parameters(ref, [zs[i]], -2, eps)
        R.zo_perturb_parameters(ref, [zs[i]], 1, eps)
        R.zo_update(ref, [zs[i]], g, lr)
        z2 = tab.export_z(s2, i)
        R.zo_perturb_parameters(ref, [z2], 1, eps)
        assert _same(ref[0], sep[i]), named[i][0]
    # fused: +1, -2, restore+update+next perturb
    with torch.no_grad():
        for (_, p), o in zip(named, other):
            p.copy_(o)
    tab.perturb(s1, 1.0, eps)
    tab.perturb(s1, -2.0, eps)
    tab.restore_update_perturb(s1, s2, eps, g, lr)
    torch.cuda.synchronize()
    bad = [named[i][0] for i, (_, p) in enumerate(named) if not _same(p.data, sep[i])]
    assert not bad, f"fused restore+update+perturb differs on {len(bad)} tensors, e.g. {bad[:3]}"
    # fused: +1, -2, restore+update, then +1
    with torch.no_grad():
        for (_, p), o in zip(named, other):
            p.copy_(o)
    tab.perturb(s1, 1.0, eps)
    tab.perturb(s1, -2.0, eps)
    tab.restore_update(s1, eps, g, lr)
    tab.perturb(s2, 1.0, eps)
    torch.cuda.synchronize()
    bad = [named[i][0] for i, (_, p) in enumerate(named) if not _same(p.data, sep[i])]
    assert not bad, f"fused restore+update differs on {len(bad)} tensors, e.g. {bad[:3]}"
    tabs.close()


def test_c5_opt30b_bf16_passes_and_projection():
    """Config C5's scale (OPT-30B bf16: 771 trainable tensors, 29.6 G elements,
    about 0.9 M tiles per launch; 96 projected groups): after +1, -2 and the
    fused restore+update+next perturb over the whole set, sampled tensors
    (first, second, middle, near the end) match the reference's expressions;
    the projection's norms, apply and reverse+norms on sampled groups match the
    reference's torch expressions with the library's norm definition."""
    from dizo_amd import _lib as L
    from dizo_amd.dizo import DiZO
    from dizo_amd.synth import build_opt
    from dizo_amd.table import ProjTable
    from dizo_amd.trainer import _ZOTables, select_trainable
    dt, eps, lr = torch.bfloat16, 1e-3, 1e-6
    g = float(torch.tensor(0.8125, dtype=dt))
    model = build_opt("opt-30b", dt, "cuda", seed=0)
    named, exclude = select_trainable(model)
    assert len(named) == 771 and sum(p.numel() for _, p in named) == 29_614_190_592
    sample = [0, 1, len(named) // 2, len(named) - 3]
    before = {i: named[i][1].detach().clone() for i in sample}
    tabs = _ZOTables(named)
    (tab, _), = tabs.tables
    s1, s2 = 2024, 2025
    tab.perturb(s1, 1.0, eps)
    tab.perturb(s1, -2.0, eps)
    tab.restore_update_perturb(s1, s2, eps, g, lr)
    torch.cuda.synchronize()
    for i in sample:
        z1, z2 = tab.export_z(s1, i), tab.export_z(s2, i)
        ref = [before[i].clone()]
        R.zo_perturb_parameters_recipe(ref, [z1], 1, eps)
        R.zo_perturb_parameters_recipe(ref, [z1], -2, eps)
        R.zo_perturb_parameters_recipe(ref, [z1], 1, eps)
        R.zo_update_recipe(ref, [z1], g, lr)
        R.zo_perturb_parameters_recipe(ref, [z2], 1, eps)
        assert _same(ref[0], named[i][1].data), named[i][0]
    del before
    tabs.close()
    names = DiZO(model, "l2norm", exclude).constraints_name
    assert len(names) == 96
    params = dict(model.named_parameters())
    th = [params[n].data for n in names]
    t0 = [(t.float() - 1e-3).to(dt) for t in th]
    ptab = ProjTable(th, t0)
    norms = torch.empty(96, dtype=dt, device="cuda")
    ptab.group_sumsq(norm_T=norms)
    gs = [0, 47, 95]
    want = torch.stack([_lib_norm(th[i] - t0[i]) for i in gs])
    assert _same(norms[gs], want)
    alpha = torch.full((96,), 0.9, dtype=dt, device="cuda")
    keep = {i: th[i].clone() for i in gs}
    ptab.project(alpha, L.DZ_PROJ_APPLY)
    ptab.project(alpha, L.DZ_PROJ_REVERSE_SUMSQ, norm_T=norms)
    torch.cuda.synchronize()
    a = alpha[:1]
    for i in gs:
        r = (keep[i] - t0[i]) * a + t0[i]
        r = (r - t0[i]) / a + t0[i]
        assert _same(th[i], r), names[i]
    want = torch.stack([_lib_norm(th[i] - t0[i]) for i in gs])
    assert _same(norms[gs], want)
    ptab.close()


def test_c4_opt13b_fp16_passes_and_projection():
    """Config C4, the headline workload (OPT-13B fp16: 643 trainable tensors,
    12,596,080,640 elements; 80 projected k/v groups): +1, -2 and the fused
    restore+update+next perturb over the whole set, then sampled tensors
    (embed_positions, the first k_proj weight, a bias, the middle tensor, the
    last) against the reference's expressions (trainer.py:1438-1442,
    1603-1608) fed the exported z; then one DiZO event's passes over all 80
    groups (trainer.py:405-451): the norms, an apply with alpha = gamma /
    (norm + 1e-8) for gamma = 0.9 of the norm, and the reverse with the norms
    of the reversed theta, on sampled groups against the reference's torch
    expressions with the library's norm definition."""
    from dizo_amd import _lib as L
    from dizo_amd.dizo import DiZO
    from dizo_amd.synth import build_opt
    from dizo_amd.table import ProjTable
    from dizo_amd.trainer import _ZOTables, select_trainable
    dt, eps, lr = torch.float16, 1e-3, 9.5e-7
    g = float(torch.tensor(-3.4375, dtype=dt))
    model = build_opt("opt-13b", dt, "cuda", seed=0)
    named, exclude = select_trainable(model)
    assert len(named) == 643 and sum(p.numel() for _, p in named) == 12_596_080_640
    names = [n for n, _ in named]
    bias = names.index("model.decoder.layers.3.self_attn.q_proj.bias")
    sample = [0, 1, bias, len(named) // 2, len(named) - 1]
    assert names[0] == "model.decoder.embed_positions.weight"
    before = {i: named[i][1].detach().clone() for i in sample}
    tabs = _ZOTables(named)
    (tab, _), = tabs.tables
    s1, s2 = 31337, 4242
    tab.perturb(s1, 1.0, eps)
    tab.perturb(s1, -2.0, eps)
    tab.restore_update_perturb(s1, s2, eps, g, lr)
    torch.cuda.synchronize()
    for i in sample:
        z1, z2 = tab.export_z(s1, i), tab.export_z(s2, i)
        ref = [before[i].clone()]
        R.zo_perturb_parameters_recipe(ref, [z1], 1, eps)
        R.zo_perturb_parameters_recipe(ref, [z1], -2, eps)
        R.zo_perturb_parameters_recipe(ref, [z1], 1, eps)
        R.zo_update_recipe(ref, [z1], g, lr)
        R.zo_perturb_parameters_recipe(ref, [z2], 1, eps)
        assert _same(ref[0], named[i][1].data), names[i]
    del before
    tabs.close()
    cname = DiZO(model, "l2norm", exclude).constraints_name
    assert len(cname) == 80
    params = dict(model.named_parameters())
    th = [params[n].data for n in cname]
    t0 = [(t.float() + 2e-3).to(dt) for t in th]
    ptab = ProjTable(th, t0)
    norms = torch.empty(80, dtype=dt, device="cuda")
    ptab.group_sumsq(norm_T=norms)
    gs = [0, 1, 39, 79]
    want = torch.stack([_lib_norm(th[i] - t0[i]) for i in gs])
    assert _same(norms[gs], want)
    gamma = (norms.float() * 0.9).to(dt)
    alpha = (gamma / (norms + 1e-8)).contiguous()  # trainer.py:464, in the model dtype
    keep = {i: th[i].clone() for i in gs}
    ptab.project(alpha, L.DZ_PROJ_APPLY)
    torch.cuda.synchronize()
    for i in gs:
        r = [keep[i].clone()]
        R.apply_constraints(r, [t0[i]], [gamma[i:i + 1]], norm=_lib_norm)
        assert _same(th[i], r[0]), cname[i]
        keep[i] = r[0]
    ptab.project(alpha, L.DZ_PROJ_REVERSE_SUMSQ, norm_T=norms)
    torch.cuda.synchronize()
    for i in gs:
        r = [keep[i]]
        R.reverse_constraints(r, [t0[i]], [alpha[i:i + 1]])
        assert _same(th[i], r[0]), cname[i]
    want = torch.stack([_lib_norm(th[i] - t0[i]) for i in gs])
    assert _same(norms[gs], want)
    ptab.close()


def _fingerprints(model) -> torch.Tensor:
    """One exact integer per parameter: the sum of its bit patterns weighted by
    (position mod 1021) + 1, in int64 (any differing element changes it unless
    the changes cancel in that weighted sum)."""
    out = []
    with torch.no_grad():
        for p in model.parameters():
            bits = _bits(p.data).reshape(-1).to(torch.int64)
            w = torch.arange(bits.numel(), device=bits.device, dtype=torch.int64) % 1021 + 1
            out.append((bits * w).sum())
            del bits, w
    return torch.stack(out).cpu()


def test_c5_opt30b_bf16_graph_replay_matches_eager():
    """Config C5's captured-graph replay (OPT-30B bf16, batch 8 x 2 candidates of
    256 tokens, the 96 projected groups' anchors on the device; the bench's
    forward: fused decoder-layer GEMMs, option-position head, SDPA): four ZO
    steps with the DiZO event (10 SPSA iterations, trainer.py:782-803) after
    the second, run eagerly and replayed from captured graphs. The losses and
    every one of the 771 trainable tensors (by exact fingerprint) agree bit
    for bit (a difference has to survive one more run of each form: the
    forward alone is not bitwise repeatable in rare cases, module doc)."""
    import gc

    from dizo_amd.synth import Cycle, build_opt, make_batches
    from dizo_amd.trainer import ZOArguments, ZOTrainer
    batches = make_batches(2, 8, 50272, seed=9, device="cuda", fixed_len=256)

    def run(graph: bool):
        model = build_opt("opt-30b", torch.bfloat16, "cuda", seed=0)
        args = ZOArguments(learning_rate=1e-6, zo_eps=1e-3, max_steps=100, enhanced="zo", zo_graph=graph,
                           zo_option_head=True, zo_fused_mlp=True, zo_fused_qkv=True)
        np.random.seed(26)
        tr = ZOTrainer(model, args, train_dataloader=Cycle(batches))
        tr.state.global_step = 48  # the event follows the update of global step 49, the second step
        it = iter(Cycle(batches))
        losses = torch.stack([tr.training_step(next(it)).reshape(()).float() for _ in range(4)])
        tr.zo_close()
        torch.cuda.synchronize()
        assert tr.dizo_trainer.i == 1
        fp = _fingerprints(model)
        out = (losses.cpu(), fp, len(list(model.parameters())))
        del tr, model
        gc.collect()
        torch.cuda.empty_cache()
        return out

    eager, graph = [run(False)], [run(True)]
    assert eager[0][2] >= 771

    def same(a, b):
        return torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])

    if not same(eager[0], graph[0]):
        # The model's forward is not bitwise repeatable in rare cases (module
        # doc): a difference counts only if it survives one more run of each
        # form, that is, if no eager run agrees with any graph run.
        eager.append(run(False))
        if not same(eager[1], graph[0]):
            graph.append(run(True))
        print("losses: eager", [e[0].tolist() for e in eager], "graph", [g[0].tolist() for g in graph], flush=True)
    le, fe, _ = eager[-1]
    lg, fg, _ = graph[-1]
    assert any(same(e, g) for e in eager for g in graph), (
        f"losses {le.tolist()} vs {lg.tolist()}; {int((fe != fg).sum())} tensors differ")
