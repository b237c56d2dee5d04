#!/usr/bin/env python3
"""DiZO zeroth-order training throughput on one MI355X.

Measures BASELINE.json's metric: ZO steps/s of the DiZO step (perturb +1,
forward, perturb -2, forward, fused restore+update, and every 50 steps the
DiZO projection event with 10 SPSA iterations on gamma) on the OPT-13B fp16
workload (config C4: 40 layers, d_model 5120, batch 16 examples x 2 candidates
of 128 random tokens, theta0 anchor resident in HBM), synthetic random-init
weights and synthetic token batches already resident in HBM. The loss's
forward computes logits only at the option positions the classification loss
reads (HF's logits_to_keep; the same loss); --full-logits computes them at
every position as the reference does. Each decoder layer's fc1 + ReLU runs as
one GEMM with a ReLU epilogue and its k/v/q projections as one GEMM (values
bit-identical to HF's layer at the C3 and C4 shapes; at C5's the fused k/v/q
GEMM runs another hipBLASLt kernel and can differ in the last bit);
--hf-layers runs HF's layer code as it is. With the fused layers, an
unpadded batch's causal attention runs through the library's MFMA kernel
(dz_attention_causal, q scaling included; not bit-identical to SDPA, within
its rounding); --sdpa keeps SDPA.

Prints one JSON line. `roofline` is the dominant library kernel (the
multi-tensor perturb / restore+update read-modify-write): algorithmic bytes
2*b*P per launch over its mean device time, measured with stream events
around every launch in the timed region. `cpu_baseline` times the
reference's expressions (the oracle's torch restatement) on the host cores
over a bounded sample and scales it to steps/s.

  python bench.py [--gpus 1] [--steps 50] [--warmup 3] [--workload c4] [--graph] [--full-logits] [--hf-layers] [--sdpa]
  python bench.py --kernels [--workload c4]     # per-pass kernel microbench (config C2 style)
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


def run_steps(wl_name: str, steps: int, warmup: int, log=print, graph: bool = False, option_head: bool = False,
              enhanced: str = "zo", fused: bool = False, attention: bool = False):
    import numpy as np
    import torch

    from dizo_amd.synth import SHAPES, Cycle, build_opt, clone_model
    from dizo_amd.timing import KernelTimer
    from dizo_amd.trainer import ZOArguments, ZOTrainer

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
    args = ZOArguments(learning_rate=1e-6, zo_eps=1e-3, max_steps=warmup + steps,
                       enhanced=None if enhanced == "none" else enhanced, zo_graph=graph, zo_option_head=option_head,
                       zo_fused_mlp=fused, zo_fused_qkv=fused, zo_fused_attention=fused and attention)
    np.random.seed(26)
    tr = ZOTrainer(model, args, train_dataloader=Cycle(batches), base_model=base)
    P = sum(p.numel() for _, p in tr.named_parameters_to_optim)
    timer = KernelTimer()
    it = iter(Cycle(batches))
    for i in range(warmup):
        tr.training_step(next(it))
    tr.zo_flush()
    torch.cuda.synchronize()
    log(f"[bench] warmup {warmup} steps done")
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
                events=sum(1 for k in range(warmup, warmup + steps) if (k + 1) % 50 == 0) if args.enhanced else 0)


def cpu_baseline(wl_name: str, log=print):
    """The reference's step on the host CPU over one decoder layer, scaled to steps/s.

    Sample: one decoder layer of the workload's shape. It times (a) the
    reference's three perturbations and its update (oracle.ref_torch: the
    expressions of trainer.py:1438-1442 and 1603-1608 with torch.normal z, in
    the model dtype) over the layer's 8 attention tensors (q/k/v/out weights
    and biases, about a third of the layer; scaled to the whole layer by
    parameter count) and (b) two forwards of one OPT decoder layer on the
    batch's hidden states (fp32: the host has no fast fp16 GEMM). A full step
    is estimated as layers x (a + b); the token embedding, LM head, loss and
    the DiZO event are left out, so the estimate flatters the CPU.
    """
    import torch

    from dizo_amd.synth import SHAPES, opt_config
    from oracle import ref_torch as R

    wl = WORKLOADS[wl_name]
    shape = SHAPES[wl["shape"]]
    dtype = _torch_dtype(wl["dtype"])
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    d, f = shape.d_model, shape.ffn
    layer_shapes = [(d, d), (d,)] * 4 + [(d,), (d,), (f, d), (f,), (d, f), (d,), (d,), (d,)]
    n_layer = sum(int(torch.Size(s).numel()) for s in layer_shapes)
    gen = torch.Generator().manual_seed(0)
    params = [(torch.randn(s, generator=gen) * 0.02).to(dtype) for s in layer_shapes[:8]]
    n_sample = sum(p.numel() for p in params)
    t0 = time.perf_counter()
    seed = 123456789
    R.zo_perturb_parameters_sampled(params, seed, 1, 1e-3)
    R.zo_perturb_parameters_sampled(params, seed, -2, 1e-3)
    R.zo_perturb_parameters_sampled(params, seed, 1, 1e-3)
    R.zo_update_sampled(params, seed, 0.5, 1e-6)
    t_zo = (time.perf_counter() - t0) * n_layer / n_sample
    log(f"[cpu] ZO passes over {n_sample} of one layer's {n_layer} params ({dtype}), scaled to the layer: "
        f"{t_zo:.2f}s on {cores} threads")
    from transformers.models.opt.modeling_opt import OPTDecoderLayer

    cfg = opt_config(shape)
    cfg._attn_implementation = "sdpa"
    layer = OPTDecoderLayer(cfg, layer_idx=0).eval()
    rows = 2 * wl["batch"]
    seq = wl["fixed_len"] or wl["max_len"]
    hidden = torch.randn(rows, seq, d, generator=gen) * 0.02
    mask = torch.full((seq, seq), float("-inf")).triu(1).reshape(1, 1, seq, seq).expand(rows, 1, seq, seq)
    with torch.inference_mode():
        layer(hidden[:2], attention_mask=mask[:2])  # warm-up
        t0 = time.perf_counter()
        for _ in range(2):
            layer(hidden, attention_mask=mask)
        t_fwd = time.perf_counter() - t0
    log(f"[cpu] two forwards of one decoder layer ({rows}x{seq} tokens, fp32): {t_fwd:.2f}s")
    step_s = shape.layers * (t_zo + t_fwd)
    return {
        "value": 1.0 / step_s,
        "unit": "steps/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"one of {shape.layers} {shape.name} decoder layers: the reference's 3 perturbations + update "
                   f"(torch.normal z, {wl['dtype']}) timed over the layer's 8 attention tensors ({n_sample} params) "
                   f"and scaled to its {n_layer} params ({t_zo:.2f}s), and 2 layer forwards on "
                   f"{rows}x{seq} tokens (fp32; {t_fwd:.2f}s), scaled x{shape.layers}; embedding, LM head, loss "
                   f"and DiZO event excluded"),
    }


def kernel_microbench(wl_name: str, reps: int = 10, log=print):
    """Per-pass GB/s of the ZO kernels over the workload's trainable set (config C2 style)."""
    import numpy as np
    import torch

    from dizo_amd.synth import SHAPES, build_opt
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
    for name, fn in cases.items():
        for tab, _ in tabs.tables:
            fn(tab)
        torch.cuda.synchronize()
        ms = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for tab, _ in tabs.tables:
                fn(tab)
            e1.record()
            torch.cuda.synchronize()
            ms.append(e0.elapsed_time(e1))
        t = float(np.median(ms))
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
        ms = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ms.append(e0.elapsed_time(e1))
        t = float(np.median(ms))
        nb = k * pbytes
        out[name] = {"ms": t, "GBps": nb / t / 1e6, "frac": nb / t / 1e6 / HBM_PEAK_GBPS, "bytes": nb}
        log(f"[kernels] {name:15s} {t:8.3f} ms {nb / t / 1e6:8.1f} GB/s")
    ptab.close()
    del t0
    # the forward's causal attention kernel at the workload's batch shape (unpadded batches only): q, k, v
    # as the fused k/v/q GEMM leaves them; algorithmic bytes = q, k, v read + output written
    from dizo_amd.attention import attention_causal, supported

    shape = SHAPES[wl["shape"]]
    hd = shape.d_model // shape.heads
    Lq = wl["fixed_len"]
    if Lq:
        n_seq, d = 2 * wl["batch"], shape.d_model
        kvq = torch.randn(n_seq, Lq, 3 * d, device="cuda", dtype=torch.float32).to(dtype)
        k, v, q = kvq.split(d, dim=-1)
        if supported(q, Lq, hd):
            fn = lambda: attention_causal(q, k, v, shape.heads, hd, hd ** -0.5)  # noqa: E731
            fn()
            torch.cuda.synchronize()
            ms = []
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                fn()
                e1.record()
                torch.cuda.synchronize()
                ms.append(e0.elapsed_time(e1))
            t = float(np.median(ms))
            nb = 4 * n_seq * Lq * d * kvq.element_size()
            out["attention"] = {"ms": t, "GBps": nb / t / 1e6, "frac": nb / t / 1e6 / HBM_PEAK_GBPS, "bytes": nb}
            log(f"[kernels] {'attention':15s} {t:8.3f} ms {nb / t / 1e6:8.1f} GB/s")
        del kvq, k, v, q
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
    return {"bytes_per_pass": nbytes, "passes": out, "calibration_copy_bytes": copy_bytes}


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
    ap.add_argument("--sdpa", action="store_true",
                    help="keep SDPA's attention (default with the fused layers: the library's causal attention "
                         "kernel for unpadded batches)")
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
    if a.kernels:
        res = kernel_microbench(a.workload, log=log)
        print(json.dumps({"metric": "ZO pass HBM GB/s", "workload": a.workload, **res}), flush=True)
        return 0
    r = run_steps(a.workload, a.steps, a.warmup, log=log, graph=a.graph, option_head=not a.full_logits,
                  enhanced=a.enhanced, fused=not a.hf_layers, attention=not a.sdpa)
    wl = WORKLOADS[a.workload]
    value = a.steps / r["elapsed"]
    summ = r["summary"]
    rmw = [summ[k] for k in ("perturb", "restore_update", "update", "restore_update_perturb") if k in summ]
    rmw_bytes = sum(s["bytes_per_launch"] * s["launches"] for s in rmw)
    rmw_ms = sum(s["total_ms"] for s in rmw)
    rmw_launches = sum(s["launches"] for s in rmw)
    achieved = rmw_bytes / (rmw_ms * 1e-3) / 1e9 if rmw_ms else None
    mean_ms = rmw_ms / rmw_launches if rmw_launches else None
    line = {
        "metric": "ZO steps/sec at OPT-13B fp16" if a.workload == "c4" else f"ZO steps/sec ({a.workload})",
        "value": value,
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": 1000.0 * r["elapsed"] / a.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"float16": "fp16", "bfloat16": "bf16", "float32": "fp32"}[wl["dtype"]],
        "data": "synthetic (random-init weights, random token batches resident in HBM)",
        "config": {"workload": f"{a.workload}: DiZO step ({wl['shape']}, {wl['dtype']}, batch {wl['batch']}x2 "
                               f"candidates, {'seq ' + str(wl['fixed_len']) if wl['fixed_len'] else 'len U[32,64]'}, "
                               f"projection every 50 steps, theta0 resident)",
                   "zo_params": r["P"], "dizo_events_timed": r["events"], "global_batch": 2 * wl["batch"],
                   "graph": a.graph, "option_head": not a.full_logits, "fused_gemms": not a.hf_layers,
                   "attention": "sdpa" if (a.hf_layers or a.sdpa) else "dz_attention_causal (unpadded batches)",
                   "enhanced": a.enhanced,
                   "seq_len": wl["fixed_len"] or wl["max_len"],
                   "device": {"name": torch.cuda.get_device_name(0),
                              "compute_units": torch.cuda.get_device_properties(0).multi_processor_count}},
        "roofline": {
            "kernel": "rmw_kernel (perturb -2 / restore+update / restore+update+next perturb)",
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS if achieved else None,
            "traffic": load_traffic("rmw_kernel", a.workload),
            "algorithmic_bytes_per_launch": rmw_bytes / rmw_launches if rmw_launches else None,
            "mean_launch_ms": mean_ms,
            "launches_per_step": rmw_launches / a.steps,
            # every library pass of the timed region (ZO passes and the DiZO
            # event's projection passes), per ZO parameter and per step
            "bytes_per_param_per_step": sum(v["bytes_per_launch"] * v["launches"] for v in summ.values())
            / (a.steps * r["P"]),
            "library_launches_per_step": sum(v["launches"] for v in summ.values()) / a.steps,
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
