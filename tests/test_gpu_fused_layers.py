"""GPU checks of the fused decoder-layer GEMMs (dizo_amd.fused_layers) on hipBLASLt.

fc1 + ReLU: at each bench workload's fc1 shape (tokens x d_model -> ffn_dim)
the GEMM with the ReLU epilogue must give the bits of HF's two kernels,
relu(linear(x)): the same GEMM, with the ReLU moved before the one rounding
to T, which it commutes with.

k/v/q: one GEMM over the [k; v; q] buffer against the three GEMMs. Where
hipBLASLt runs the same kernel family for both shapes (OPT-125m fp32,
OPT-2.7B and OPT-13B fp16) the bits must agree. At OPT-30B bf16 the fused
shape's q block comes out of another accumulation order (a few thousand of
29 M elements differ, all near zero, where cancellation leaves few
significant bits): each element must stay within one unit in the last place
of T plus the fp32 dot-product error bound K * 2^-24 * sum |x_i w_i|.

Then ZO runs through the trainer, with a DiZO event (its projection table is
built after the weights moved), fused against unfused, bit for bit.
"""
import copy

import numpy as np
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().contiguous().view({2: torch.int16, 4: torch.int32}[t.element_size()])


def _ulp(x: torch.Tensor) -> torch.Tensor:
    """Unit in the last place of T at each element's magnitude."""
    p = {torch.float16: 11, torch.bfloat16: 8, torch.float32: 24}[x.dtype]
    emin = {torch.float16: -14, torch.bfloat16: -126, torch.float32: -126}[x.dtype]
    _, e = torch.frexp(x.float().abs())
    return torch.ldexp(torch.ones_like(x, dtype=torch.float32), (e - 1).clamp_min(emin) - (p - 1))


# (tokens, d_model, ffn_dim, dtype): C4 (OPT-13B), C3's padded token counts
# (OPT-2.7B, 32 sequences of 40-72 tokens), C5 (OPT-30B), C1 (OPT-125m), tiny
FC1_SHAPES = [
    (4096, 5120, 20480, torch.float16),
    (1280, 2560, 10240, torch.float16),
    (1792, 2560, 10240, torch.float16),
    (2304, 2560, 10240, torch.float16),
    (4096, 7168, 28672, torch.bfloat16),
    (1536, 768, 3072, torch.float32),
    (24, 64, 256, torch.bfloat16),
]


@pytest.mark.parametrize("m,k,n,dt", FC1_SHAPES)
def test_fused_fc1_bits_at_workload_shapes(m, k, n, dt):
    from dizo_amd.fused_layers import ReluLinear

    print(f"[fused fc1] {m}x{k}->{n} {dt}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(m + n)
    lin = torch.nn.Linear(k, n, device="cuda", dtype=dt)
    with torch.no_grad():
        lin.weight.normal_(0.0, 0.02, generator=g)
        lin.bias.normal_(0.0, 0.02, generator=g)
    x = torch.randn(m, k, device="cuda", dtype=dt, generator=g)
    with torch.inference_mode():
        want = torch.relu(F.linear(x, lin.weight, lin.bias))
        lin.__class__ = ReluLinear
        got = lin(x)
        got3 = lin(x.view(32 if m % 32 == 0 else 1, -1, k)).view(m, n)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(want)), f"{(got != want).sum().item()} elements differ"
    assert torch.equal(_bits(got3), _bits(want))


# (tokens, d_model, dtype, bit-identical expected)
QKV_SHAPES = [
    (4096, 5120, torch.float16, True),
    (1280, 2560, torch.float16, True),
    (1792, 2560, torch.float16, True),
    (2304, 2560, torch.float16, True),
    (4096, 7168, torch.bfloat16, False),
    (1536, 768, torch.float32, True),
]


@pytest.mark.parametrize("m,d,dt,exact", QKV_SHAPES)
def test_fused_kvq_gemm_at_workload_shapes(m, d, dt, exact):
    print(f"[fused kvq] {m}x{d} {dt}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(m + d)
    x = torch.randn(m, d, device="cuda", dtype=dt, generator=g)
    w = torch.randn(3 * d, d, device="cuda", dtype=dt, generator=g) * 0.02
    b = torch.randn(3 * d, device="cuda", dtype=dt, generator=g) * 0.02
    with torch.inference_mode():
        sep = [F.linear(x, w[i * d:(i + 1) * d], b[i * d:(i + 1) * d]) for i in range(3)]
        fused = F.linear(x, w, b).split(d, dim=-1)
    for i, (name, s, f) in enumerate(zip("kvq", sep, fused)):
        if exact:
            assert torch.equal(_bits(s), _bits(f)), f"{name}: {(s != f).sum().item()} elements differ"
        else:
            with torch.inference_mode():
                scale = F.linear(x.float().abs(), w[i * d:(i + 1) * d].float().abs(),
                                 b[i * d:(i + 1) * d].float().abs())
            bigger = torch.maximum(s.float().abs(), f.float().abs()).to(dt)
            bound = _ulp(bigger) + d * 2.0 ** -24 * scale
            diff = (s.float() - f.float()).abs()
            assert bool((diff <= bound).all()), f"{name}: max diff {diff.max().item()}"
            assert (diff > 0).float().mean().item() < 1e-3


def _run(model, batches, fused: bool, enhanced):
    from dizo_amd.synth import Cycle
    from dizo_amd.trainer import ZOArguments, ZOTrainer

    np.random.seed(31)
    args = ZOArguments(learning_rate=1e-3, zo_eps=1e-3, max_steps=len(batches), enhanced=enhanced,
                       zo_fused_mlp=fused, zo_fused_qkv=fused, zo_option_head=True)
    tr = ZOTrainer(model, args, train_dataloader=Cycle(batches[:4]) if enhanced else None)
    losses = torch.stack([tr.training_step(b) for b in batches])
    tr.zo_flush()
    gam = [g.detach().clone() for g in tr.dizo_trainer.dizo.constraints] if enhanced else []
    tr.zo_close()
    return losses, gam


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("enhanced", [None, "zo"])
def test_trainer_fused_layers_bit_identical(dt, enhanced):
    from dizo_amd.fused_layers import FusedQKVOPTAttention
    from dizo_amd.synth import build_opt, make_batches

    print(f"[fused trainer] {dt} enhanced={enhanced}", flush=True)
    model_a = build_opt("opt-tiny", dt, "cuda", seed=8)
    model_b = copy.deepcopy(model_a)
    batches = make_batches(50 if enhanced else 6, 4, 512, seed=9, device="cuda", min_len=8, max_len=20)
    la, ga = _run(model_a, batches, True, enhanced)
    lb, gb = _run(model_b, batches, False, enhanced)
    assert type(model_a.model.decoder.layers[0].self_attn) is FusedQKVOPTAttention
    assert torch.equal(_bits(la), _bits(lb)), (la - lb).abs().max().item()
    for x, y in zip(ga, gb):
        assert torch.equal(_bits(x), _bits(y))
    pb = dict(model_b.named_parameters())
    for n, p in model_a.named_parameters():
        assert torch.equal(_bits(p), _bits(pb[n])), n
