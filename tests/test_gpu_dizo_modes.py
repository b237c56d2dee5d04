"""The projection with the ratio or gamma supplied, the searched-ratio (grid)
event, and config C1 (one MeZO step and a fixed-ratio projection at
OPT-125m fp32 against the CPU oracle's arithmetic)."""
import copy

import numpy as np
import pytest
import torch

from oracle import arith as A
from oracle import ref_torch as R

pytestmark = pytest.mark.gpu

DTS = [torch.float16, torch.bfloat16, torch.float32]
DTNAME = {torch.float16: A.F16, torch.bfloat16: A.BF16, torch.float32: A.F32}


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().view({2: torch.int16, 4: torch.int32}[t.element_size()])


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(_bits(a), _bits(b))


def _lib_norm(t: torch.Tensor) -> torch.Tensor:
    s = (t.double() ** 2).sum().float()
    return torch.sqrt(s.double()).float().to(t.dtype)


def _pair(dt, seed=13, shape="opt-tiny"):
    """Two identical models moved away from their (identical) anchors, and the anchors."""
    from dizo_amd.synth import build_opt
    model_a = build_opt(shape, dt, "cuda", seed=seed)
    anchor = copy.deepcopy(model_a)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    with torch.no_grad():
        for p in model_a.parameters():
            p.add_((torch.randn(p.shape, device="cuda", generator=gen) * 1e-2).to(dt))
    return model_a, copy.deepcopy(model_a), anchor


def _dizo(anchor):
    from dizo_amd.dizo import DiZO
    from dizo_amd.trainer import select_trainable
    _, exclude = select_trainable(anchor)
    return DiZO(anchor, "l2norm", exclude)


@pytest.mark.parametrize("dt", DTS)
def test_supplied_ratio_matches_reference_expression(dt):
    """apply_ratio: theta0 + alpha (theta - theta0) with alpha supplied (one value,
    then one per group) against (new - anchor) * alpha + anchor in torch."""
    model_a, model_b, anchor = _pair(dt)
    dz = _dizo(anchor)
    names = dz.constraints_name
    dz.apply_ratio(model_a, anchor, 0.9)
    pb, p0 = dict(model_b.named_parameters()), dict(anchor.named_parameters())
    a09 = torch.tensor([0.9], dtype=torch.float32).to(dt).cuda()
    with torch.no_grad():
        for n in names:
            pb[n].copy_((pb[n] - p0[n]) * a09 + p0[n])
    pa = dict(model_a.named_parameters())
    assert all(_same(pa[n].data, pb[n].data) for n in pa)
    ratios = [0.5 + 0.5 * i / max(1, len(names) - 1) for i in range(len(names))]
    dz.apply_ratio(model_a, anchor, ratios)
    with torch.no_grad():
        for n, r in zip(names, ratios):
            a = torch.tensor([r], dtype=torch.float32).to(dt).cuda()
            pb[n].copy_((pb[n] - p0[n]) * a + p0[n])
    assert all(_same(pa[n].data, pb[n].data) for n in pa)
    dz.close()


@pytest.mark.parametrize("dt", DTS)
def test_supplied_gamma_matches_reference(dt):
    """apply_gamma with fp32 target norms (the reference's constraint Parameters
    are fp32: alpha fp32, one rounding at the end) against apply_constraints of
    trainer.py:405-436 written with torch, fed the same gammas."""
    model_a, model_b, anchor = _pair(dt, seed=14)
    dz = _dizo(anchor)
    names = dz.constraints_name
    gam = [0.05 * (1 + i) for i in range(len(names))]
    dz.apply_gamma(model_a, anchor, gam)
    pb, p0 = dict(model_b.named_parameters()), dict(anchor.named_parameters())
    cons = [torch.tensor([g], dtype=torch.float32, device="cuda") for g in gam]
    R.apply_constraints([pb[n] for n in names], [p0[n] for n in names], cons, norm=_lib_norm)
    pa = dict(model_a.named_parameters())
    bad = [n for n in pa if not _same(pa[n].data, pb[n].data)]
    assert not bad, bad[:3]
    dz.close()


def _grid_case(dt, shape, batch, seed):
    """The searched ratio (ENHANCED=grid) on `shape`: for each of 8 ratios in
    [0.5, 1.0] the reference procedure takes a deep copy, applies the ratio
    to every projected tensor and evaluates the loss with the oracle's
    restatement of the reference's forward wrap (trainer.py:470-542); the
    lowest wins and is applied. The library's in-place search must give the
    same losses, the same choice and the same weights, bit for bit."""
    model_a, model_b, anchor = _pair(dt, seed=seed, shape=shape)
    dz = _dizo(anchor)
    names = dz.constraints_name
    cands = tuple(np.linspace(0.5, 1.0, 8))
    model_a.eval()
    r, losses = dz.grid_search(model_a, anchor, batch, cands)
    p0 = dict(anchor.named_parameters())
    ref_losses = []
    for c in cands:
        m = copy.deepcopy(model_b).eval()
        pm = dict(m.named_parameters())
        a = torch.tensor([c], dtype=torch.float32).to(dt).cuda()
        with torch.no_grad():
            for n in names:
                pm[n].copy_((pm[n] - p0[n]) * a + p0[n])
            ref_losses.append(R.forward_wrap_with_option_len(m, **batch).float())
        del m
    assert all(_same(x, y.reshape(())) for x, y in zip(losses, ref_losses)), (losses, ref_losses)
    best = int(torch.stack(ref_losses).argmin())
    assert r == float(cands[best])
    pb = dict(model_b.named_parameters())
    a = torch.tensor([cands[best]], dtype=torch.float32).to(dt).cuda()
    with torch.no_grad():
        for n in names:
            pb[n].copy_((pb[n] - p0[n]) * a + p0[n])
    pa = dict(model_a.named_parameters())
    assert all(_same(pa[n].data, pb[n].data) for n in pa)
    dz.close()
    return len(names), [float(x) for x in losses], r


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_grid_search_matches_reference_procedure(dt):
    from dizo_amd.synth import make_batches
    batch = make_batches(1, 4, 512, seed=9, device="cuda", min_len=8, max_len=20)[0]
    _grid_case(dt, "opt-tiny", batch, 15)


def test_c3_shape_grid_search_matches_reference_procedure():
    """The grid event at config C3's shape (OPT-2.7B fp16, 64 k/v groups, one
    batch of 16 x 2 candidates of length U[32, 64])."""
    from dizo_amd.synth import make_batches
    batch = make_batches(1, 16, 50272, seed=29, device="cuda", min_len=32, max_len=64)[0]
    groups, losses, r = _grid_case(torch.float16, "opt-2.7b", batch, 17)
    print(f"C3 grid: {groups} groups, losses {losses}, ratio {r}", flush=True)
    assert groups == 64


def test_c1_mezo_step_and_fixed_ratio_projection_match_cpu_oracle():
    """Config C1: OPT-125m fp32 (195 trainable tensors, 86.6 M elements), one
    MeZO step (eps 1e-3, lr 1e-6, seed from np.random) and a projection of the
    k/v tensors with the ratio fixed at 0.9, on the GPU; against the CPU
    oracle's arithmetic (oracle.arith, numpy) fed the exported z, the step's
    projected gradient and the schedule's lr: every element bit for bit. The
    step's loss is the float64 brute force's on the same weights within 1e-5."""
    from dizo_amd.synth import PAD_ID, build_opt, make_batch
    from dizo_amd.trainer import ZOArguments, ZOTrainer, select_trainable
    from oracle import loss as OL
    dt, eps, lr0 = torch.float32, 1e-3, 1e-6
    model = build_opt("opt-125m", dt, "cuda", seed=1)
    init = {n: p.detach().cpu().numpy().view(np.uint32).copy() for n, p in model.named_parameters()}
    anchor = copy.deepcopy(model)
    batch = make_batch(16, 50272, gen=torch.Generator().manual_seed(3), min_len=32, max_len=64, device="cuda")
    np.random.seed(26)
    tr = ZOTrainer(model, ZOArguments(learning_rate=lr0, zo_eps=eps, max_steps=1, enhanced=None))
    loss = float(tr.training_step(batch))
    tr.zo_flush()
    seed, g = tr.zo_random_seed, tr.projected_grad
    named, _ = select_trainable(model)
    assert len(named) == 195
    dz = _dizo(anchor)
    dz.apply_ratio(model, anchor, 0.9)
    torch.cuda.synchronize()
    lr = A.zo_lr(lr0, 0, 1)
    alpha = A.from_f32(np.float32(0.9), A.F32)
    proj = set(dz.constraints_name)
    for n, p in named:
        z = tr.export_z(n, seed).cpu().numpy().view(np.uint32)
        th = init[n].ravel()
        for s in (1, -2, 1):
            th = A.perturb(th, z.ravel(), s, eps, A.F32)
        th = A.update(th, z.ravel(), g, lr, A.F32)
        if n in proj:
            th = A.apply(th, init[n].ravel(), alpha, A.F32)
        got = p.detach().cpu().numpy().view(np.uint32).ravel()
        assert np.array_equal(got, th), n
    with torch.no_grad():
        m0 = build_opt("opt-125m", dt, "cuda", seed=1).eval()
        named0 = dict(m0.named_parameters())
        for n in init:
            named0[n].data.copy_(torch.from_numpy(init[n].view(np.float32)).reshape(named0[n].shape))
        zs = {n: tr.export_z(n, seed) for n, _ in named}
        for n, _ in named:
            named0[n].data.add_(zs[n] * np.float32(eps))  # the +eps z weights the step's first loss is taken at
        logits = m0(input_ids=batch["input_ids"], attention_mask=batch["attention_mask"]).logits
    want = OL.classification_loss(logits.double().cpu().numpy(), batch["input_ids"].cpu().numpy(),
                                  batch["labels"].tolist(), batch["option_len"].tolist(),
                                  batch["num_options"].tolist(), PAD_ID)
    assert loss == pytest.approx(want, rel=1e-5)
    dz.close()
    tr.zo_close()
