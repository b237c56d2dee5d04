"""The reference's hot-path expressions written with torch ops (test oracle only).

Each function evaluates the same torch expression the reference evaluates,
in the same operand order, but takes z (and, for DiZO, the gamma noise and
the losses) as inputs instead of drawing them from torch's generator. Run on
CPU it pins ``oracle.arith`` against torch's real CPU kernels; run on the
ROCm device (GPU box) it pins the HIP kernels against torch's device kernels,
which is what the reference executes. On CPU it is also the timed CPU
baseline of the reference's step (``bench.py``).
"""
from __future__ import annotations

from typing import Callable, Sequence

import torch


def zo_perturb_parameters(params: Sequence[torch.Tensor], zs: Sequence[torch.Tensor],
                          scaling_factor: float, zo_eps: float) -> None:
    """trainer.py:1438-1442 with z supplied: param.data = param.data + s * z * eps."""
    for param, z in zip(params, zs):
        param.data = param.data + scaling_factor * z * zo_eps


def zo_update(params: Sequence[torch.Tensor], zs: Sequence[torch.Tensor], projected_grad: float,
              lr: float) -> None:
    """trainer.py:1603-1608 with z supplied: param.data = param.data - lr * (g * z)."""
    for param, z in zip(params, zs):
        param.data = param.data - lr * (projected_grad * z)


def _f32(x: float) -> float:
    """A Python scalar as torch's kernels use it with a 16-bit or fp32 tensor:
    converted to the fp32 "opmath" type."""
    return float(torch.tensor(x, dtype=torch.float32))


def _rt(x64: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """An exactly computed float64 value rounded as torch's CPU and CUDA kernels
    round an fp32-opmath result: to fp32 (the op), then to the tensor dtype."""
    return x64.float().to(dtype)


def zo_perturb_parameters_recipe(params: Sequence[torch.Tensor], zs: Sequence[torch.Tensor],
                                 scaling_factor: float, zo_eps: float) -> None:
    """trainer.py:1438-1442 with z supplied, each operation evaluated exactly in
    float64 and rounded as torch's CPU and CUDA kernels round it (fp32 result,
    then the parameter dtype): R(p + R(R(s * z) * eps)).

    Products of a 16-bit (or fp32) value and an fp32 scalar are exact in
    float64, so this is the recipe itself on any device. It exists for device
    runs: on some launch paths (seen on tensors of 1 and 2,560 elements, not
    on 1M) ROCm torch's 16-bit `scalar * tensor` kernel rounds the exact
    product to the 16-bit type once, which differs from the recipe when the
    fp32 product falls exactly halfway between two 16-bit values (a rare tie;
    torch on the CPU and CUDA rounds the tie to even from the fp32 product)."""
    s, eps = _f32(scaling_factor), _f32(zo_eps)
    for param, z in zip(params, zs):
        dt = param.dtype
        a = _rt(z.double() * s, dt)
        b = _rt(a.double() * eps, dt)
        param.data = _rt(param.data.double() + b.double(), dt)


def zo_update_recipe(params: Sequence[torch.Tensor], zs: Sequence[torch.Tensor], projected_grad: float,
                     lr: float) -> None:
    """trainer.py:1603-1608 with z supplied, in the recipe form of
    zo_perturb_parameters_recipe: R(p - R(lr * R(g * z)))."""
    g, lr32 = _f32(projected_grad), _f32(lr)
    for param, z in zip(params, zs):
        dt = param.dtype
        c = _rt(z.double() * g, dt)
        d = _rt(c.double() * lr32, dt)
        param.data = _rt(param.data.double() - d.double(), dt)


def zo_perturb_parameters_sampled(params: Sequence[torch.Tensor], seed: int, scaling_factor: float,
                                  zo_eps: float) -> None:
    """trainer.py:1438-1442 verbatim, z drawn by torch.normal (the CPU-baseline workload)."""
    torch.manual_seed(seed)
    for param in params:
        z = torch.normal(mean=0, std=1, size=param.data.size(), device=param.data.device,
                         dtype=param.data.dtype)
        param.data = param.data + scaling_factor * z * zo_eps


def zo_update_sampled(params: Sequence[torch.Tensor], seed: int, projected_grad: float, lr: float) -> None:
    """trainer.py:1603-1608 verbatim (torch.normal z)."""
    torch.manual_seed(seed)
    for param in params:
        z = torch.normal(mean=0, std=1, size=param.data.size(), device=param.data.device,
                         dtype=param.data.dtype)
        param.data = param.data - lr * (projected_grad * z)


def projected_grad(loss1: torch.Tensor, loss2: torch.Tensor, zo_eps: float) -> float:
    """trainer.py:1587."""
    return ((loss1 - loss2) / (2 * zo_eps)).item()


def project_ratio(new: torch.Tensor, anchor: torch.Tensor, constraint: torch.Tensor,
                  norm: Callable = torch.norm) -> torch.Tensor:
    """trainer.py:453-465 (l2norm mode). `norm` is torch.norm in the reference;
    tests may inject another evaluation of the same norm."""
    t = new.detach() - anchor.detach()
    norms = norm(t)
    return constraint / (norms + 1e-8)


def apply_constraints(news: Sequence[torch.Tensor], anchors: Sequence[torch.Tensor],
                      constraints: Sequence[torch.Tensor], norm: Callable = torch.norm) -> list:
    """trainer.py:405-436 over the projected tensors; returns the alphas."""
    alphas = []
    for new_para, anchor_para, c in zip(news, anchors, constraints):
        alpha = project_ratio(new_para, anchor_para, c, norm)
        alphas.append(alpha)
        v = (new_para.detach() - anchor_para.detach()) * alpha
        temp = v + anchor_para.detach()
        with torch.no_grad():
            new_para.copy_(temp)
    return alphas


def reverse_constraints(news: Sequence[torch.Tensor], anchors: Sequence[torch.Tensor],
                        alphas: Sequence[torch.Tensor]) -> None:
    """trainer.py:439-451."""
    for new_para, anchor_para, alpha in zip(news, anchors, alphas):
        v = (new_para.detach() - anchor_para.detach()) / alpha
        temp = v + anchor_para.detach()
        with torch.no_grad():
            new_para.copy_(temp)


def dizo_zo_iteration(news, anchors, gammas: list, init: bool, z_gamma: Sequence[torch.Tensor],
                      loss_fn: Callable[[int], torch.Tensor], norm: Callable = torch.norm):
    """One ZO gamma iteration, trainer.py:564-614, with the gamma noise and the
    two losses supplied (loss_fn(k) is the k-th forward's loss, k = 0, 1).

    gammas: list of per-group gamma tensors (updated in place of the list).
    Returns (ts, loss1, loss2).
    """
    with torch.no_grad():
        ts = [norm(p.data - a.data) for p, a in zip(news, anchors)]
        if init:
            for i in range(len(gammas)):
                gammas[i] = ts[i]
        tau, zo_eps, step_size = 0.2, 0.1, 2
        zs = []
        for i in range(len(gammas)):  # perturb_gamma(1, ...), trainer.py:553-560
            z = torch.clip(z_gamma[i], (-tau / zo_eps) * ts[i], (tau / zo_eps) * ts[i])
            zs.append(z)
            gammas[i] = gammas[i] + 1 * z * zo_eps
        alphas = apply_constraints(news, anchors, gammas, norm)
        loss1 = loss_fn(0)
        reverse_constraints(news, anchors, alphas)
        for i in range(len(gammas)):
            gammas[i] = gammas[i] + -2 * zs[i] * zo_eps
        alphas = apply_constraints(news, anchors, gammas, norm)
        loss2 = loss_fn(1)
        reverse_constraints(news, anchors, alphas)
        for i in range(len(gammas)):
            gammas[i] = gammas[i] + 1 * zs[i] * zo_eps
        grad = (loss1 - loss2) / (2 * zo_eps)
        for i in range(len(gammas)):
            gammas[i] = torch.clip(gammas[i] - step_size * ts[i] * grad * zs[i], (1 - tau) * ts[i],
                                   (1 + tau) * ts[i])
    return ts, loss1, loss2


def option_loss(logits, input_ids, labels, option_len, num_options, pad_id: int) -> torch.Tensor:
    """trainer.py:495-528 (the classification branch of
    forward_wrap_with_option_len, also trainer.py:1466-1508) on given logits:
    shift, the per-row option masking loop, log_softmax over the vocabulary,
    the option-position log-probability mean, then the cross-entropy over
    each example's candidates."""
    import torch.nn.functional as F

    shift_logits = logits[..., :-1, :].contiguous()
    shift_labels = torch.clone(input_ids)[..., 1:].contiguous()
    shift_labels[shift_labels == pad_id] = -100
    for i, n in enumerate(option_len.tolist()):
        shift_labels[i, :-n] = -100
    loss_fct = torch.nn.CrossEntropyLoss(ignore_index=-100)
    log_probs = F.log_softmax(shift_logits, dim=-1)
    mask = shift_labels != -100
    shift_labels[~mask] = 0
    selected = torch.gather(log_probs, dim=-1, index=shift_labels.unsqueeze(-1)).squeeze(-1)
    selected = (selected * mask).sum(-1) / mask.sum(-1)
    nopt = num_options.tolist()
    if any(x != nopt[0] for x in nopt):
        loss, start, count = 0, 0, 0
        while start < len(nopt):
            end = start + nopt[start]
            loss = loss_fct(selected[start:end].unsqueeze(0), labels[start:end][0].unsqueeze(0)) + loss
            count += 1
            start = end
        return loss / count
    return loss_fct(selected.view(-1, nopt[0]), labels.view(-1, nopt[0])[:, 0])


def forward_loss(model, input_ids, attention_mask, labels, option_len, num_options, pad_id: int) -> torch.Tensor:
    """trainer.py:1446-1522 (classification branch) with torch ops: the full
    logits of a forward without gradients, then option_loss. The CPU
    baseline's forward and loss."""
    with torch.no_grad():
        logits = model(input_ids=input_ids, attention_mask=attention_mask).logits
    return option_loss(logits, input_ids, labels, option_len, num_options, pad_id)


def forward_wrap_with_option_len(model, input_ids=None, labels=None, option_len=None, num_options=None,
                                 **kwargs) -> torch.Tensor:
    """DiZO.forward_wrap_with_option_len, trainer.py:470-542 (classification
    branch), as the first-order DiZO path calls it: the model's forward with
    autograd enabled (full logits), then option_loss with the model's own pad
    id (trainer.py:501). Returns the loss."""
    logits = model(input_ids=input_ids, **kwargs).logits
    return option_loss(logits, input_ids, labels, option_len, num_options, model.config.pad_token_id)


def dizo_fo_objective(model, anchors: dict, names: Sequence[str], gammas: Sequence[torch.Tensor], data: dict):
    """DiZO.forward with apply=False, trainer.py:714-741: a deep copy of the
    model in eval mode, apply_constraints on it (trainer.py:405-436, every
    parameter's requires_grad cleared, alpha = gamma / (torch.norm(Delta) +
    1e-8) per projected tensor, the copy_ recorded by autograd), the loss of
    forward_wrap_with_option_len and 1e-3 * sum |gamma|.

    anchors: name -> theta0 tensor; names: the projected tensors in the order
    of the gamma Parameters. Returns (pgm_loss, vs, deltas, denominators): the
    differentiable v = Delta * alpha of each group (retain_grad() set) and
    its Delta and norm + 1e-8, for the gradient bound of a test (v.grad is
    kept when gamma requires a gradient)."""
    import copy

    cm = copy.deepcopy(model)
    cm.eval()
    for p in cm.parameters():
        p.requires_grad = False
    named = dict(cm.named_parameters())
    vs, deltas, denoms = [], [], []
    for g, n in zip(gammas, names):
        new_para, anchor_para = named[n], anchors[n]
        t = new_para.detach() - anchor_para.detach()
        denom = torch.norm(t) + 1e-8
        alpha = g / denom
        v = (new_para.detach() - anchor_para.detach()) * alpha
        if v.requires_grad:
            v.retain_grad()
        temp = v + anchor_para.detach()
        new_para.copy_(temp)
        vs.append(v)
        deltas.append(t)
        denoms.append(denom.detach())
    loss = forward_wrap_with_option_len(cm, **data)
    pgm_loss = loss + 1e-3 * sum(p.abs().sum() for p in gammas)
    return pgm_loss, vs, deltas, denoms


def dizo_fo_apply(model, anchors: dict, names: Sequence[str], gammas: Sequence[torch.Tensor]) -> None:
    """DiZO.forward with apply=True, trainer.py:720-725 (apply_constraints in
    place under no_grad, trainer.py:428-433)."""
    named = dict(model.named_parameters())
    with torch.no_grad():
        for g, n in zip(gammas, names):
            new_para, anchor_para = named[n], anchors[n]
            alpha = g / (torch.norm(new_para.detach() - anchor_para.detach()) + 1e-8)
            temp = (new_para.detach() - anchor_para.detach()) * alpha + anchor_para.detach()
            new_para.copy_(temp)


def dizo_fo_event(model, anchors: dict, names: Sequence[str], batches: Sequence[dict], max_iters: int = 10,
                  proj_lr: float = 0.1):
    """dizo_trainer.dizo_iters, trainer.py:805-830: one fp32 gamma Parameter
    per projected tensor, created as torch.Tensor([0]) (trainer.py:388-403),
    Adam(lr = proj_lr) (trainer.py:758), max_iters iterations of the
    objective, backward and step, each on the next batch, then the final
    apply. Returns (gammas as one fp32 tensor, the iterations' losses)."""
    dev = next(model.parameters()).device
    gammas = [torch.nn.Parameter(torch.Tensor([0]).to(dev)) for _ in names]
    opt = torch.optim.Adam(gammas, lr=proj_lr)
    losses = []
    for it in range(max_iters):
        pgm, _, _, _ = dizo_fo_objective(model, anchors, names, gammas, batches[it % len(batches)])
        losses.append(float(pgm.detach()))
        opt.zero_grad()
        pgm.backward()
        opt.step()
    dizo_fo_apply(model, anchors, names, gammas)
    return torch.cat([g.detach().reshape(1) for g in gammas]), losses


def zo_step_sampled(model, params: Sequence[torch.Tensor], batch: dict, seed: int, zo_eps: float,
                    pad_id: int):
    """trainer.py:1570-1595 verbatim (torch.normal z): +1, loss1, -2, loss2,
    projected_grad, +1. Returns (loss1, projected_grad)."""
    zo_perturb_parameters_sampled(params, seed, 1, zo_eps)
    loss1 = forward_loss(model, pad_id=pad_id, **batch)
    zo_perturb_parameters_sampled(params, seed, -2, zo_eps)
    loss2 = forward_loss(model, pad_id=pad_id, **batch)
    g = projected_grad(loss1, loss2, zo_eps)
    zo_perturb_parameters_sampled(params, seed, 1, zo_eps)
    return loss1, g


def apply_ratio(news: Sequence[torch.Tensor], anchors: Sequence[torch.Tensor], alpha: float) -> None:
    """trainer.py:428-436 with the ratio supplied (alpha in place of
    constraint / (norm + 1e-8)): new <- (new - anchor) * alpha + anchor."""
    for new_para, anchor_para in zip(news, anchors):
        v = (new_para.detach() - anchor_para.detach()) * alpha
        temp = v + anchor_para.detach()
        with torch.no_grad():
            new_para.copy_(temp)
