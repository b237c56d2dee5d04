#!/usr/bin/env python3
"""DiZO zeroth-order training throughput on one MI355X.

Measures BASELINE.json's metric: ZO steps/s of the DiZO step (perturb +1,
forward, perturb -2, forward, fused restore+update, and every 50 steps the
DiZO projection event with 10 SPSA iterations on gamma) on the OPT-13B fp16
workload (config C4: 40 layers, d_model 5120, batch 16 examples x 2 candidates
of 128 random tokens, theta0 anchor resident in HBM), synthetic random-init
weights and synthetic token batches already resident in HBM.

Every timed window holds at least one DiZO event: the trainer's step counter
starts where the event (after the update of every 50th step,
trainer.py:1611) falls on the window's last step (on steps 49, 99, ... of the
window when --steps exceeds 50). `value` is the amortised rate, one event per
50 steps: steps / (t_steps + t_event * steps / 50), with t_event the mean
timed event and t_steps the window's time without its events; the plain ZO
step rate and the event time are reported beside it.

The forward stays on PyTorch-ROCm: SDPA's attention and HF's decoder layers,
with two GEMM-level fusions that give HF's values bit for bit at the bench
shapes (fc1 + ReLU as one GEMM with a ReLU epilogue; k/v/q as one GEMM), and
logits computed only at the option positions the classification loss reads
(HF's logits_to_keep; the same loss). --full-logits computes them at every
position as the reference does; --hf-layers runs HF's layer code as it is.

Prints one JSON line. `roofline` is the dominant library kernel (the
multi-tensor perturb / restore+update read-modify-write): algorithmic bytes
2*b*P per launch over its mean device time, measured for every launch in the
timed region with a stream-event pair that the runtime records as the kernel
starts and ends (hipExtLaunchKernel, through dz_table_time_next), so the
host's launch work is not counted; the rocprofv3 kernel trace of the same
command agrees with it. `cpu_baseline` times the
reference's expressions (the oracle's torch restatement) on the host cores:
the whole step at C1, a sampled and scaled step otherwise.

  python bench.py [--gpus 1] [--steps 50] [--warmup 3] [--workload c4] [--graph] [--full-logits] [--hf-layers]
  python bench.py --kernels [--workload c2|c4]  # per-pass kernel microbench (config C2: OPT-2.7B fp16)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0

WORKLOADS = {
    # BASELINE.json configs; c4 is the one the metric is quoted on
    "c1": dict(shape="opt-125m", dtype="float32", batch=16, min_len=32, max_len=64, fixed_len=None),
    # C2 is kernel-only (--kernels): the ZO passes over OPT-2.7B's fp16 trainable set
    "c2": dict(shape="opt-2.7b", dtype="float16", batch=16, min_len=32, max_len=64, fixed_len=None,
               kernels_only=True),
    "c3": dict(shape="opt-2.7b", dtype="float16", batch=16, min_len=32, max_len=64, fixed_len=None),
    "c4": dict(shape="opt-13b", dtype="float16", batch=16, min_len=None, max_len=None, fixed_len=128),
    "c5": dict(shape="opt-30b", dtype="bfloat16", batch=8, min_len=None, max_len=None, fixed_len=256),
}


def _torch_dtype(name):
    import torch

    return {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[name]


def _batches(wl, n, vocab, device):
    from dizo_amd.synth import make_batches

    kw = dict(fixed_len=wl["fixed_len"]) if wl["fixed_len"] else dict(min_len=wl["min_len"], max_len=wl["max_len"])
    return make_batches(n, wl["batch"], vocab, seed=1, device=device, **kw)


def load_traffic(kernel: str, workload: str):
    """HBM bytes per launch measured by rocprofv3 PMC runs (profiles/traffic.json), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data.get(workload, {}).get(kernel)
    except (OSError, ValueError):
        return None


def event_offset(steps: int, warmup: int, interval: int = 50) -> int:
    """Global step the trainer starts from, so that the DiZO event (after the
    update of every `interval`-th step, trainer.py:1611) falls on timed step
    min(steps, interval) - 1 of the window (and every `interval` steps after)."""
    first = min(steps, interval) - 1
    return (interval - 1 - (warmup + first)) % interval


def run_steps(wl_name: str, steps: int, warmup: int, log=print, graph: bool = False, option_head: bool = False,
              enhanced: str = "zo", fused: bool = False, host_grad: bool = False):
    import numpy as np
    import torch

    from dizo_amd.synth import SHAPES, Cycle, build_opt, clone_model
    from dizo_amd.timing import KernelTimer
    from dizo_amd.trainer import DIZO_INTERVAL, ZOArguments, ZOTrainer

    wl = WORKLOADS[wl_name]
    dtype = _torch_dtype(wl["dtype"])
    shape = SHAPES[wl["shape"]]
    t0 = time.perf_counter()
    model = build_opt(shape, dtype, "cuda", seed=0)
    base = clone_model(model)
    batches = _batches(wl, 8, shape.vocab, "cuda")
    torch.cuda.synchronize()
    log(f"[bench] built {shape.name} {dtype} + anchor in {time.perf_counter() - t0:.1f}s; "
        f"mem {torch.cuda.memory_allocated() / 2**30:.1f} GiB")
    offset = event_offset(steps, warmup, DIZO_INTERVAL) if enhanced != "none" else 0
    args = ZOArguments(learning_rate=1e-6, zo_eps=1e-3, max_steps=offset + warmup + steps,
                       enhanced=None if enhanced == "none" else enhanced, zo_graph=graph, zo_option_head=option_head,
                       zo_fused_mlp=fused, zo_fused_qkv=fused,
                       zo_host_grad=host_grad)
    np.random.seed(26)
    tr = ZOTrainer(model, args, train_dataloader=Cycle(batches), base_model=base)
    # start the step counter at `offset` (the LR schedule follows it, trainer.py:1100-1102)
    tr.state.global_step = offset
    tr.lr_scheduler.step()
    P = sum(p.numel() for _, p in tr.named_parameters_to_optim)
    # every DiZO event is timed on its own (device synchronised on both sides)
    event_s = []
    dizo_event = tr._dizo_event

    def timed_event(m, seed):
        torch.cuda.synchronize()
        t = time.perf_counter()
        dizo_event(m, seed)
        torch.cuda.synchronize()
        event_s.append(time.perf_counter() - t)

    tr._dizo_event = timed_event
    timer = KernelTimer()
    it = iter(Cycle(batches))
    for i in range(warmup):
        tr.training_step(next(it))
    tr.zo_flush()
    torch.cuda.synchronize()
    log(f"[bench] warmup {warmup} steps done (from global step {offset}; {len(event_s)} DiZO events)")
    event_s.clear()
    tr.kernel_timer = timer
    if getattr(tr, "dizo_trainer", None) is not None and args.enhanced:
        tr.dizo_trainer.dizo.kernel_timer = timer
    t_start = time.perf_counter()
    for i in range(steps):
        tr.training_step(next(it))
    tr.zo_flush()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    losses = [float(x) for x in tr.loss_list[-steps:]]
    summary = timer.summary()
    tr.zo_close()
    return dict(elapsed=elapsed, P=P, summary=summary, losses=losses, elem_bytes=torch.finfo(dtype).bits // 8,
                events=len(event_s), event_s=list(event_s), offset=offset)


def amortised(steps: int, elapsed: float, event_s, interval: int = 50):
    """(steps/s with one event per `interval` steps, ZO steps/s without events,
    mean event seconds): steps / (t_steps + t_event * steps / interval)."""
    t_ev = sum(event_s)
    t_steps = elapsed - t_ev
    if not event_s:
        return steps / elapsed, steps / elapsed, None
    mean_ev = t_ev / len(event_s)
    return steps / (t_steps + mean_ev * steps / interval), steps / t_steps, mean_ev


ZO_PASSES = ("perturb", "update", "restore_update", "restore_update_perturb")


def amortised_passes(summ: dict, steps: int, events: int, P: int, pass_bytes: float, interval: int = 50) -> dict:
    """Library launches and bytes per ZO parameter per step with one DiZO
    event per `interval` steps, as `value` amortises the event's time.

    A steady step makes two read-modify-write launches (the -2 perturbation
    and the fused restore + update + next perturbation). An event adds its
    projection passes and changes the ZO launches around it (the restore +
    update before it and the +1 perturbation after it are launches of their
    own); both are measured in the window per event and spread over
    `interval` steps. Without events the window's own per-step figures are
    returned. pass_bytes: the algorithmic bytes of one RMW launch (2 b P).
    Replays of captured steps are not timed; without a timed steady pass the
    ZO launches are counted from the step's structure instead: two per step
    and one more per event (the restore + update before it), as the eager
    step launches them."""
    zo = [v for k, v in summ.items() if k in ZO_PASSES]
    ev = [v for k, v in summ.items() if k not in ZO_PASSES]
    if "restore_update_perturb" in summ or "perturb" in summ:
        zo_launches = sum(v["launches"] for v in zo)
        zo_bytes = sum(v["bytes_per_launch"] * v["launches"] for v in zo)
    else:
        zo_launches = 2 * steps + events
        zo_bytes = zo_launches * pass_bytes
    if not events:
        return {"bytes_per_param_per_step": (zo_bytes + sum(v["bytes_per_launch"] * v["launches"] for v in ev))
                / (steps * P),
                "library_launches_per_step": (zo_launches + sum(v["launches"] for v in ev)) / steps,
                "event_amortisation": None}
    zo_extra_launches = (zo_launches - 2 * steps) / events
    zo_extra_bytes = (zo_bytes - 2 * steps * pass_bytes) / events
    ev_launches = sum(v["launches"] for v in ev) / events
    ev_bytes = sum(v["bytes_per_launch"] * v["launches"] for v in ev) / events
    return {
        "bytes_per_param_per_step": (2 * pass_bytes + (zo_extra_bytes + ev_bytes) / interval) / P,
        "library_launches_per_step": 2 + (zo_extra_launches + ev_launches) / interval,
        "event_amortisation": {"interval_steps": interval, "launches_per_event": ev_launches + zo_extra_launches,
                               "bytes_per_event": ev_bytes + zo_extra_bytes},
    }


def _cpu_threads() -> int:
    """Uses every host core this process may run on; returns the count."""
    import torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return cores


def _median_s(fn, reps: int = 3, warm: int = 1) -> float:
    """Median wall time of fn() over `reps` runs after `warm` untimed runs."""
    import statistics

    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return float(statistics.median(ts))


def _cpu_kv_sample(shape, dtype, gen):
    """One decoder layer's k_proj and v_proj weights (2 d^2 elements) in the
    model dtype, and perturbed anchors: the sample the CPU legs time."""
    import torch

    d = shape.d_model
    ws = [(torch.randn(d, d, generator=gen) * 0.02).to(dtype) for _ in range(2)]
    anchors = [(w.float() + 1e-3 * torch.randn(d, d, generator=gen)).to(dtype) for w in ws]
    return ws, anchors


def _cpu_pass_times(params, anchors, reps: int = 3) -> dict:
    """Median seconds of each pass of the reference over `params` (its
    expressions with torch.normal z, oracle.ref_torch): perturb +1 / -2 /
    restore +1 (trainer.py:1438-1442), update (trainer.py:1603-1608), and the
    projection's norm (trainer.py:455-457), apply (405-436, gamma 0.9 of the
    norm) and reverse (439-451)."""
    import torch

    from oracle import ref_torch as R

    seed = 123456789
    ps = [torch.nn.Parameter(p.clone(), requires_grad=False) for p in params]
    out = {
        "perturb+1": _median_s(lambda: R.zo_perturb_parameters_sampled(ps, seed, 1, 1e-3), reps),
        "perturb-2": _median_s(lambda: R.zo_perturb_parameters_sampled(ps, seed, -2, 1e-3), reps),
        "restore+1": _median_s(lambda: R.zo_perturb_parameters_sampled(ps, seed, 1, 1e-3), reps),
        "update": _median_s(lambda: R.zo_update_sampled(ps, seed, 0.5, 1e-6), reps),
        "proj_norm": _median_s(lambda: [torch.norm(p.detach() - a) for p, a in zip(ps, anchors)], reps),
    }
    gam = [0.9 * torch.norm(p.detach() - a) for p, a in zip(ps, anchors)]
    alphas = []

    def apply():
        alphas[:] = R.apply_constraints(ps, anchors, gam)

    out["proj_apply"] = _median_s(apply, reps)
    out["proj_reverse"] = _median_s(lambda: R.reverse_constraints(ps, anchors, alphas), reps)
    return out


# algorithmic bytes per element of each pass, in units of the element size
_PASS_BYTES = {"perturb+1": 2, "perturb-2": 2, "restore+1": 2, "update": 2, "proj_norm": 2, "proj_apply": 3,
               "proj_reverse": 3}


def cpu_baseline_kernels(wl_name: str, log=print) -> dict:
    """The reference's per-pass expressions on the host cores (the CPU leg of
    the kernel microbench): median of 3 runs of each pass over one decoder
    layer's k_proj and v_proj weights of the workload's shape, GB/s from the
    same algorithmic bytes as the GPU passes."""
    import torch

    from dizo_amd.synth import SHAPES

    wl = WORKLOADS[wl_name]
    shape = SHAPES[wl["shape"]]
    dtype = _torch_dtype(wl["dtype"])
    cores = _cpu_threads()
    ws, anchors = _cpu_kv_sample(shape, dtype, torch.Generator().manual_seed(0))
    n = sum(w.numel() for w in ws)
    eb = ws[0].element_size()
    t = _cpu_pass_times(ws, anchors)
    passes = {k: {"s": v, "GBps": _PASS_BYTES[k] * eb * n / v / 1e9} for k, v in t.items()}
    for k, v in passes.items():
        log(f"[cpu] {k:13s} {v['s'] * 1e3:9.1f} ms {v['GBps']:7.2f} GB/s ({n} {wl['dtype']} elements, {cores} threads)")
    return {
        "value": passes["perturb+1"]["GBps"],
        "unit": "GB/s (perturb pass)",
        "cores": cores,
        "kind": "port",
        "sample": (f"one {shape.name} decoder layer's k_proj and v_proj weights ({n} {wl['dtype']} elements); "
                   f"median of 3 runs after 1 warm-up per pass"),
        "passes": passes,
    }


def cpu_baseline_c1(log=print) -> dict:
    """Config C1 on the host cores, whole: the reference's MeZO step
    (oracle.ref_torch.zo_step_sampled: trainer.py:1570-1595 with torch.normal
    z, full-logit forwards and the option-masked loss of trainer.py:1446-1522)
    and update (trainer.py:1597-1608) on an OPT-125m fp32 model, batch 16 x 2
    candidates of length U[32, 64], followed by the DiZO projection with the
    ratio 0.9 on every k/v tensor (trainer.py:428-436). Median of 3 steps after
    1 warm-up; per-pass times from the same model."""
    import copy

    import torch
    from transformers import OPTForCausalLM

    from dizo_amd.synth import PAD_ID, SHAPES, make_batch, opt_config
    from oracle import ref_torch as R

    wl = WORKLOADS["c1"]
    cores = _cpu_threads()
    torch.manual_seed(0)
    model = OPTForCausalLM(opt_config(SHAPES[wl["shape"]])).eval()
    named = [(n, p) for n, p in model.named_parameters() if p.requires_grad]
    named = [(n, p) for n, p in named if n != "model.decoder.embed_tokens.weight"]  # trainer.py:1160
    params = [p for _, p in named]
    kv = [p for n, p in named if n.endswith(("self_attn.k_proj.weight", "self_attn.v_proj.weight"))]
    anchors = [p.detach().clone() for p in kv]
    batch = make_batch(wl["batch"], SHAPES[wl["shape"]].vocab, gen=torch.Generator().manual_seed(1),
                       min_len=wl["min_len"], max_len=wl["max_len"])
    P = sum(p.numel() for p in params)
    seeds = iter(range(1000, 2000))

    def step():
        seed = next(seeds)
        _, g = R.zo_step_sampled(model, params, batch, seed, 1e-3, PAD_ID)
        R.zo_update_sampled(params, seed, g, 1e-6)
        R.apply_ratio(kv, anchors, 0.9)

    with torch.inference_mode():
        t_step = _median_s(step)
        t_fwd = _median_s(lambda: R.forward_loss(model, pad_id=PAD_ID, **batch))
        t_perturb = _median_s(lambda: R.zo_perturb_parameters_sampled(params, 7, 1, 1e-3))
        t_update = _median_s(lambda: R.zo_update_sampled(params, 7, 0.5, 1e-6))
        t_apply = _median_s(lambda: R.apply_ratio(kv, anchors, 0.9))
    Pk = sum(p.numel() for p in kv)
    log(f"[cpu] c1 step {t_step:.3f}s (forward {t_fwd:.3f}s, perturb {t_perturb:.3f}s, update {t_update:.3f}s, "
        f"projection {t_apply:.4f}s) on {cores} threads")
    del model, copy
    return {
        "value": 1.0 / t_step,
        "unit": "steps/s",
        "cores": cores,
        "kind": "port",
        "sample": ("the whole C1 step (MeZO step, update and the 0.9 projection) on an OPT-125m fp32 model, "
                   "batch 16x2 of length U[32,64]; median of 3 steps after 1 warm-up"),
        "passes": {
            "forward": {"s": t_fwd},
            "perturb": {"s": t_perturb, "GBps": 8 * P / t_perturb / 1e9},
            "update": {"s": t_update, "GBps": 8 * P / t_update / 1e9},
            "proj_apply_ratio": {"s": t_apply, "GBps": 12 * Pk / t_apply / 1e9},
        },
    }


def cpu_baseline_sampled(wl_name: str, log=print) -> dict:
    """The reference's step on the host cores, estimated from timed samples
    (the whole C3-C5 step takes minutes on the CPU; the line labels the
    result "estimate" and carries the measured passes, GB/s of the sample,
    beside it):
      * the four ZO passes (trainer.py:1438-1442 x3, 1603-1608; torch.normal
        z, model dtype) over one decoder layer's k_proj and v_proj weights,
        scaled to the whole trainable set by parameter count;
      * two forwards of one OPT decoder layer on the batch's hidden states
        (fp32: the host has no fast fp16 GEMM), x layers;
      * the full-logit LM head GEMM of one forward (fp32);
      * the DiZO event (trainer.py:782-803, every 50 steps): 20 forwards,
        21 applies and 20 reverses of the projection, amortised per step, the
        projection passes timed on the same k/v sample and scaled to every
        layer's k/v.
    Each factor is reported in the line. The embedding lookup and the loss's
    log_softmax are left out."""
    import torch

    from dizo_amd.synth import SHAPES, opt_config

    wl = WORKLOADS[wl_name]
    shape = SHAPES[wl["shape"]]
    dtype = _torch_dtype(wl["dtype"])
    cores = _cpu_threads()
    gen = torch.Generator().manual_seed(0)
    d, f, Lyr = shape.d_model, shape.ffn, shape.layers
    n_layer = 4 * d * d + 4 * d + 2 * d + f * d + f + d * f + d + 2 * d  # attention, norms, MLP
    P = Lyr * n_layer + (shape.max_positions + 2) * d + 2 * d  # + learned positions, final norm
    ws, anchors = _cpu_kv_sample(shape, dtype, gen)
    n_kv = sum(w.numel() for w in ws)
    t = _cpu_pass_times(ws, anchors, reps=1)
    t_zo = (t["perturb+1"] + t["perturb-2"] + t["restore+1"] + t["update"]) * P / n_kv
    t_event_proj = Lyr * (21 * t["proj_apply"] + 20 * t["proj_reverse"])
    from transformers.models.opt.modeling_opt import OPTDecoderLayer

    cfg = opt_config(shape)
    cfg._attn_implementation = "sdpa"
    layer = OPTDecoderLayer(cfg, layer_idx=0).eval()
    rows = 2 * wl["batch"]
    seq = wl["fixed_len"] or wl["max_len"]
    hidden = torch.randn(rows, seq, d, generator=gen) * 0.02
    mask = torch.full((seq, seq), float("-inf")).triu(1).reshape(1, 1, seq, seq).expand(rows, 1, seq, seq)
    head = torch.randn(shape.vocab, d, generator=gen) * 0.02
    with torch.inference_mode():
        layer(hidden[:2], attention_mask=mask[:2])  # warm-up
        t0 = time.perf_counter()
        for _ in range(2):
            layer(hidden, attention_mask=mask)
        t_fwd2 = time.perf_counter() - t0
        t0 = time.perf_counter()
        torch.matmul(hidden.reshape(-1, d), head.t())
        t_head = time.perf_counter() - t0
    fwd_per_step = 2 + 20 / 50
    step_s = t_zo + Lyr * t_fwd2 / 2 * fwd_per_step + t_head * fwd_per_step + t_event_proj / 50
    eb = ws[0].element_size()
    measured = {k: {"s": v, "GBps": _PASS_BYTES[k] * eb * n_kv / v / 1e9} for k, v in t.items()}
    log(f"[cpu] {wl_name}: ZO passes {t_zo:.1f}s (sampled {n_kv} of {P} params), layer forwards x2 "
        f"{t_fwd2:.2f}s, LM head {t_head:.2f}s, event projection {t_event_proj:.1f}s per event; "
        f"{step_s:.1f}s per step on {cores} threads")
    return {
        "value": 1.0 / step_s,
        "unit": "steps/s",
        "cores": cores,
        # an extrapolation from the measured samples below, not a measured step
        "kind": "estimate",
        "measured_passes": measured,
        "sample": (f"estimated from timed samples: the 4 ZO passes ({wl['dtype']}, torch.normal z) over one "
                   f"{shape.name} layer's k/v weights ({n_kv} params) scaled to P={P}; 2 forwards of one decoder "
                   f"layer ({rows}x{seq} tokens, fp32) x {Lyr} layers; the full-logit LM head (fp32); the DiZO "
                   f"event's 20 forwards and 41 projection passes per 50 steps"),
        "factors": {"zo_pass_scale": P / n_kv, "layers": Lyr, "forwards_per_step": fwd_per_step,
                    "event_projection_passes_per_step": 41 / 50, "event_included": True},
        "components_s": {"zo_passes": t_zo, "layer_forward_x2": t_fwd2, "lm_head": t_head,
                         "event_projection": t_event_proj, "step": step_s},
    }


def cpu_baseline(wl_name: str, log=print) -> dict:
    """The CPU baseline of a full-step bench line: the whole step at C1, the
    sampled estimate at C3-C5."""
    return cpu_baseline_c1(log) if wl_name == "c1" else cpu_baseline_sampled(wl_name, log)


def kernel_microbench(wl_name: str, reps: int = 10, log=print):
    """Per-pass GB/s of the ZO kernels over the workload's trainable set (config C2 style)."""
    import numpy as np
    import torch

    from dizo_amd.synth import SHAPES, build_opt
    from dizo_amd.timing import KernelTimer
    from dizo_amd.trainer import _ZOTables, select_trainable

    wl = WORKLOADS[wl_name]
    dtype = _torch_dtype(wl["dtype"])
    model = build_opt(SHAPES[wl["shape"]], dtype, "cuda", seed=0)
    named, _ = select_trainable(model)
    tabs = _ZOTables(named)
    nbytes = tabs.bytes_per_pass
    out = {}
    g = float(np.float32(np.random.default_rng(0).standard_normal()))
    cases = {
        "perturb+1": lambda t: t.perturb(26, 1.0, 1e-3),
        "perturb-2": lambda t: t.perturb(26, -2.0, 1e-3),
        "restore+1": lambda t: t.perturb(26, 1.0, 1e-3),
        "update": lambda t: t.update(26, g, 1e-6),
        "restore_update": lambda t: t.restore_update(26, 1e-3, g, 1e-6),
        "restore_update_perturb": lambda t: t.restore_update_perturb(26, 27, 1e-3, g, 1e-6),
    }
    # each launch timed from its first kernel's start to its last kernel's end (KernelTimer with tables)
    timer = KernelTimer()
    zo_tables = [tab for tab, _ in tabs.tables]
    for name, fn in cases.items():
        for tab in zo_tables:
            fn(tab)
        torch.cuda.synchronize()
        for _ in range(reps):
            with timer.span(name, nbytes, zo_tables):
                for tab in zo_tables:
                    fn(tab)
            torch.cuda.synchronize()
        t = float(np.median([a.elapsed_time(b) for a, b, _ in timer.spans[name]]))
        out[name] = {"ms": t, "GBps": nbytes / t / 1e6, "frac": nbytes / t / 1e6 / HBM_PEAK_GBPS}
        log(f"[kernels] {name:15s} {t:8.3f} ms {nbytes / t / 1e6:8.1f} GB/s")
    tabs.close()
    # projection passes over the projected (k/v) tensors, theta0 a perturbed copy
    from dizo_amd import _lib as L
    from dizo_amd.dizo import DiZO
    from dizo_amd.table import ProjTable

    _, exclude = select_trainable(model)
    names = DiZO(model, "l2norm", exclude).constraints_name
    params = dict(model.named_parameters())
    th = [params[n].data for n in names]
    t0 = [(t.float() + 1e-3).to(t.dtype) for t in th]
    ptab = ProjTable(th, t0)
    G = len(names)
    alpha = torch.full((G,), 0.9, dtype=dtype, device="cuda")
    norms = torch.empty(G, dtype=dtype, device="cuda")
    pbytes = ptab.bytes_per_tensor_pass
    proj_cases = {
        "proj_sumsq": (2, lambda: ptab.group_sumsq(norm_T=norms)),
        "proj_apply": (3, lambda: ptab.project(alpha, L.DZ_PROJ_APPLY)),
        "proj_reverse_sumsq": (3, lambda: ptab.project(alpha, L.DZ_PROJ_REVERSE_SUMSQ, norm_T=norms)),
    }
    for name, (k, fn) in proj_cases.items():
        fn()
        torch.cuda.synchronize()
        for _ in range(reps):
            with timer.span(name, k * pbytes, [ptab]):
                fn()
            torch.cuda.synchronize()
        t = float(np.median([a.elapsed_time(b) for a, b, _ in timer.spans[name]]))
        nb = k * pbytes
        out[name] = {"ms": t, "GBps": nb / t / 1e6, "frac": nb / t / 1e6 / HBM_PEAK_GBPS, "bytes": nb}
        log(f"[kernels] {name:15s} {t:8.3f} ms {nb / t / 1e6:8.1f} GB/s")
    ptab.close()
    del t0
    # calibration for counter-based traffic: a plain device copy of known size
    # (reads and writes copy_bytes each), launched twice
    copy_bytes = 4 << 30
    src = torch.empty(copy_bytes // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    # context: the same copy timed (reads and writes copy_bytes: a plain streaming RMW's traffic pattern)
    ms = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    t = float(np.median(ms))
    out["device_copy_4GiB"] = {"ms": t, "GBps": 2 * copy_bytes / t / 1e6, "frac": 2 * copy_bytes / t / 1e6 / HBM_PEAK_GBPS}
    log(f"[kernels] device copy 4 GiB {t:8.3f} ms {2 * copy_bytes / t / 1e6:8.1f} GB/s")
    del src, dst
    # context: PyTorch's own in-place elementwise kernel over 16 GiB (x ^= 0 on int32: every byte read and
    # written once, the RMW passes' traffic pattern with no arithmetic), a practical streaming ceiling
    ip_bytes = 16 << 30
    buf = torch.zeros(ip_bytes // 4, dtype=torch.int32, device="cuda")
    buf.bitwise_xor_(0)
    torch.cuda.synchronize()
    ms = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        buf.bitwise_xor_(0)
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    del buf
    t = float(np.median(ms))
    out["torch_inplace_16GiB"] = {"ms": t, "GBps": 2 * ip_bytes / t / 1e6, "frac": 2 * ip_bytes / t / 1e6 / HBM_PEAK_GBPS}
    log(f"[kernels] torch in-place xor 16 GiB {t:8.3f} ms {2 * ip_bytes / t / 1e6:8.1f} GB/s")
    eb = torch.finfo(dtype).bits // 8
    # one ZO step of the reference (trainer.py:1580-1608): +1, -2, +1 and the update, 4 read-modify-write
    # passes; fused: +1, -2 and restore+update (3); across steps: -2 and restore+update+next perturb (2)
    steps = {"separate": 4, "restore_update_fused": 3, "next_perturb_fused": 2}
    return {"bytes_per_pass": nbytes, "passes": out, "calibration_copy_bytes": copy_bytes,
            "launches_per_step": steps,
            "bytes_per_param_per_step": {k: 2 * eb * v for k, v in steps.items()}}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="c4", choices=sorted(WORKLOADS))
    ap.add_argument("--kernels", action="store_true", help="per-pass kernel microbench instead of full steps")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true", help="replay each ZO step as a captured hipGraph")
    ap.add_argument("--enhanced", default="zo", choices=["zo", "fo", "grid", "none"],
                    help="DiZO event every 50 steps: ZO gamma search (the reference's dizo.sh), first-order, "
                         "ratio grid, or none (MeZO)")
    ap.add_argument("--full-logits", action="store_true",
                    help="compute logits at every position, as the reference does (default: only at the option "
                         "positions the loss reads, the same loss)")
    ap.add_argument("--hf-layers", action="store_true",
                    help="run HF's decoder layer code as it is (default: fc1 + ReLU as one GEMM with a ReLU "
                         "epilogue, k/v/q as one GEMM; the same values at the bench shapes)")
    ap.add_argument("--host-grad", action="store_true",
                    help="read projected_grad back to the host in every step, as the reference does (default: the "
                         "kernels read it on the device and the step has no synchronisation; the same values)")
    a = ap.parse_args(argv)
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the DiZO step path is measured on a "
                                   "single MI355X (multi-GPU sharding is a design note, not a code path)",
                          "n_gpus": a.gpus}), flush=True)
        return 2

    def log(msg):
        print(msg, file=sys.stderr, flush=True)

    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}), flush=True)
        return 1
    from dizo_amd import _lib

    _lib.load()
    if WORKLOADS[a.workload].get("kernels_only") and not a.kernels:
        print(json.dumps({"error": f"workload {a.workload} is a kernel microbench: add --kernels"}), flush=True)
        return 2
    if a.kernels:
        res = kernel_microbench(a.workload, log=log)
        line = {"metric": "ZO pass HBM GB/s", "workload": a.workload, **res}
        if not a.no_cpu_baseline:
            try:
                line["cpu_baseline"] = cpu_baseline_kernels(a.workload, log=log)
            except Exception as e:  # reported, not fatal: the GPU measurement stands
                line["cpu_baseline"] = {"error": f"{type(e).__name__}: {e}"}
        print(json.dumps(line), flush=True)
        return 0
    r = run_steps(a.workload, a.steps, a.warmup, log=log, graph=a.graph, option_head=not a.full_logits,
                  enhanced=a.enhanced, fused=not a.hf_layers, host_grad=a.host_grad)
    wl = WORKLOADS[a.workload]
    value, zo_rate, event_s = amortised(a.steps, r["elapsed"], r["event_s"])
    summ = r["summary"]
    # the dominant library kernel: the fused restore + update + next perturbation
    # (one launch per steady step, the longest), else the plain perturbation
    dom_name = "restore_update_perturb" if "restore_update_perturb" in summ else "perturb"
    dom = summ.get(dom_name)
    achieved = dom["GBps"] if dom else None
    rmw = [summ[k] for k in ("perturb", "restore_update", "update", "restore_update_perturb") if k in summ]
    rmw_bytes = sum(s["bytes_per_launch"] * s["launches"] for s in rmw)
    rmw_ms = sum(s["total_ms"] for s in rmw)
    rmw_launches = sum(s["launches"] for s in rmw)
    line = {
        "metric": "ZO steps/sec at OPT-13B fp16" if a.workload == "c4" else f"ZO steps/sec ({a.workload})",
        "value": value,
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": 1000.0 / value,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"float16": "fp16", "bfloat16": "bf16", "float32": "fp32"}[wl["dtype"]],
        "data": "synthetic (random-init weights, random token batches resident in HBM)",
        "config": {"workload": f"{a.workload}: DiZO step ({wl['shape']}, {wl['dtype']}, batch {wl['batch']}x2 "
                               f"candidates, {'seq ' + str(wl['fixed_len']) if wl['fixed_len'] else 'len U[32,64]'}, "
                               f"projection every 50 steps, theta0 resident)",
                   "zo_params": r["P"], "dizo_events_timed": r["events"], "global_batch": 2 * wl["batch"],
                   "first_global_step": r["offset"],
                   "graph": a.graph, "option_head": not a.full_logits, "fused_gemms": not a.hf_layers,
                   "attention": "sdpa",
                   "enhanced": a.enhanced, "projected_grad": "host (.item())" if a.host_grad else "device",
                   "seq_len": wl["fixed_len"] or wl["max_len"],
                   "device": {"name": torch.cuda.get_device_name(0),
                              "compute_units": torch.cuda.get_device_properties(0).multi_processor_count}},
        "timing": {
            # value = steps / (t_steps + t_event * steps / 50): one DiZO event per 50 steps
            "timed_region_s": r["elapsed"],
            "zo_steps_per_s_without_events": zo_rate,
            "dizo_event_s": event_s,
            "dizo_event_s_all": r["event_s"],
        },
        "roofline": {
            "kernel": f"rmw_kernel ({dom_name.replace('_', ' + ')})",
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS if achieved else None,
            "traffic": load_traffic("rmw_kernel", a.workload),
            "algorithmic_bytes_per_launch": dom["bytes_per_launch"] if dom else None,
            "mean_launch_ms": dom["mean_ms"] if dom else None,
            "launch_timing": "kernel start/end events (hipExtLaunchKernel)",
            # all read-modify-write launches of the window together
            "rmw_all": {"GBps": rmw_bytes / (rmw_ms * 1e-3) / 1e9 if rmw_ms else None,
                        "frac": rmw_bytes / (rmw_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS if rmw_ms else None,
                        "launches_per_step": rmw_launches / a.steps},
            # every library pass, per ZO parameter and per step, with the DiZO
            # event amortised one per 50 steps as in `value` (amortised_passes)
            **amortised_passes(summ, a.steps, r["events"], r["P"], 2 * r["elem_bytes"] * r["P"]),
        },
        "kernels": summ,
        "loss_first_last": [r["losses"][0], r["losses"][-1]] if r["losses"] else None,
    }
    if not a.no_cpu_baseline:
        try:
            line["cpu_baseline"] = cpu_baseline(a.workload, log=log)
        except Exception as e:  # reported, not fatal: the GPU measurement stands
            line["cpu_baseline"] = {"error": f"{type(e).__name__}: {e}"}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
