"""GPU checks of the causal attention kernel (dizo_amd.attention, dz_attention_causal).

What pins it: an fp32 reference of the same definition (q rounded to T after
HF's scaling, causal softmax, P @ V, all in fp32 on contiguous operands), and
torch's own SDPA flash kernel on the same inputs, whose error against that
reference sets the scale. The kernel rounds P to T before the product with
V, as the flash kernel does, so its error must be of the same size: within
a small multiple of SDPA's, and within an absolute bound per dtype. Inputs
come as the fused k/v/q GEMM leaves them: strided views of one buffer.
"""
import math

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _kvq(n_seq, L, H, hd, dt, seed, std=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    kvq = torch.randn(n_seq, L, 3 * H * hd, device="cuda", dtype=torch.float32, generator=g) * std
    return kvq.to(dt)


def _reference(q, k, v, H, hd, scale):
    """fp32 attention with q = R_T(q * scale), as HF computes q before SDPA."""
    n_seq, L, _ = q.shape
    qs = (q.float() * scale).to(q.dtype).float()
    qh = qs.view(n_seq, L, H, hd).transpose(1, 2).contiguous()
    kh = k.float().view(n_seq, L, H, hd).transpose(1, 2).contiguous()
    vh = v.float().view(n_seq, L, H, hd).transpose(1, 2).contiguous()
    s = torch.matmul(qh, kh.transpose(-1, -2).contiguous())
    mask = torch.ones(L, L, dtype=torch.bool, device=q.device).triu(1)
    s = s.masked_fill(mask, float("-inf"))
    o = torch.matmul(torch.softmax(s, dim=-1), vh)
    return o.transpose(1, 2).contiguous(), qh.to(q.dtype), kh.to(q.dtype), vh.to(q.dtype)


CASES = [
    (4, 128, 40, 128, torch.float16),   # C4's attention (fewer sequences)
    (2, 256, 7, 128, torch.bfloat16),   # C5's length and head dim
    (3, 64, 5, 64, torch.float16),
    (2, 32, 3, 64, torch.bfloat16),
    (2, 96, 4, 128, torch.float16),     # odd number of 32-query blocks
    (1, 192, 2, 128, torch.bfloat16),   # 6 blocks: pairs on 3 waves
    (2, 160, 3, 64, torch.float16),     # 5 blocks: pairs + the middle block
]


@pytest.mark.parametrize("n_seq,L,H,hd,dt", CASES)
def test_attention_matches_fp32_reference(n_seq, L, H, hd, dt):
    from dizo_amd.attention import attention_causal

    print(f"[attention] n_seq={n_seq} L={L} H={H} hd={hd} {dt}", flush=True)
    kvq = _kvq(n_seq, L, H, hd, dt, seed=L + H)
    d = H * hd
    k, v, q = kvq.split(d, dim=-1)
    scale = hd ** -0.5
    out = attention_causal(q, k, v, H, hd, scale)
    torch.cuda.synchronize()
    ref, qh, kh, vh = _reference(q, k, v, H, hd, scale)
    with torch.inference_mode():
        sdpa = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True, scale=1.0).transpose(1, 2).float()
    err = (out.float() - ref).abs().max().item()
    err_sdpa = (sdpa - ref).abs().max().item()
    bound = {torch.float16: 4e-3, torch.bfloat16: 3e-2}[dt]
    print(f"  max|out - ref| {err:.3g}, max|sdpa - ref| {err_sdpa:.3g}", flush=True)
    assert out.shape == (n_seq, L, H, hd)
    assert math.isfinite(err) and err <= bound
    assert err <= 2.0 * err_sdpa + bound / 4


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_attention_large_scores_stay_finite_and_accurate(dt):
    """q and k of standard deviation 6: scaled scores reach about +-100, far
    outside exp's range without the running-max subtraction. The output must
    stay finite and as close to the fp32 reference as SDPA's."""
    from dizo_amd.attention import attention_causal

    n_seq, L, H, hd = 2, 128, 4, 128
    kvq = _kvq(n_seq, L, H, hd, dt, seed=21, std=6.0)
    d = H * hd
    k, v, q = kvq.split(d, dim=-1)
    scale = hd ** -0.5
    out = attention_causal(q, k, v, H, hd, scale)
    ref, qh, kh, vh = _reference(q, k, v, H, hd, scale)
    with torch.inference_mode():
        sdpa = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True, scale=1.0).transpose(1, 2).float()
    assert bool(torch.isfinite(out).all())
    err = (out.float() - ref).abs().max().item()
    err_sdpa = (sdpa - ref).abs().max().item()
    print(f"[attention large] {dt}: max|out - ref| {err:.3g}, max|sdpa - ref| {err_sdpa:.3g}", flush=True)
    assert err <= 2.0 * err_sdpa + 1e-3


def test_attention_first_query_is_its_value_row():
    """Query 0 sees only key 0: its output is v[0] rounded to T (softmax weight exactly 1)."""
    from dizo_amd.attention import attention_causal

    kvq = _kvq(2, 64, 4, 64, torch.float16, seed=9)
    k, v, q = kvq.split(256, dim=-1)
    out = attention_causal(q, k, v, 4, 64, 0.125)
    assert torch.equal(out[:, 0].reshape(2, -1), v[:, 0])


def test_attention_rejects_bad_arguments():
    from dizo_amd import _lib as L
    from dizo_amd.attention import attention_causal

    kvq = _kvq(2, 64, 2, 64, torch.float16, seed=1)
    k, v, q = kvq.split(128, dim=-1)
    with pytest.raises(L.DzError, match="L must be"):
        attention_causal(q[:, :48], k[:, :48], v[:, :48], 2, 64, 0.125)
    with pytest.raises(L.DzError, match="head_dim"):
        attention_causal(q, k, v, 4, 32, 0.125)
    out = torch.empty(2 * 64 * 128, dtype=torch.float16, device="cuda")
    strides = (q.stride(1), k.stride(1), v.stride(1), q.stride(0), k.stride(0), v.stride(0))
    with pytest.raises(L.DzError, match="aligned"):
        L.call("dz_attention_causal", 1, q.data_ptr() + 2, k.data_ptr(), v.data_ptr(), out.data_ptr(), *strides,
               2, 64, 2, 64, 0.125, None)
    with pytest.raises(L.DzError, match="overlaps"):
        L.call("dz_attention_causal", 1, q.data_ptr(), k.data_ptr(), v.data_ptr(), kvq.data_ptr(), *strides,
               2, 64, 2, 64, 0.125, None)
    with pytest.raises(L.DzError, match="strides"):
        L.call("dz_attention_causal", 1, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
               100, k.stride(1), v.stride(1), q.stride(0), k.stride(0), v.stride(0), 2, 64, 2, 64, 0.125, None)
    with pytest.raises(L.DzError, match="dtype"):
        L.call("dz_attention_causal", 0, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), *strides,
               2, 64, 2, 64, 0.125, None)


def _mini(dt, seed=3):
    from dizo_amd.synth import build_opt

    return build_opt("opt-mini", dt, "cuda", seed=seed)  # head_dim 64, vocab 4096


def _loss(model, batch):
    from dizo_amd.trainer import forward_wrap_with_option_len

    with torch.inference_mode():
        return forward_wrap_with_option_len(model, **batch, return_dict=True).loss.float().item()


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_model_loss_with_library_attention_close_to_sdpa(dt):
    import copy

    from dizo_amd.fused_layers import fuse_forward
    from dizo_amd.synth import make_batches

    print(f"[attention model] {dt}", flush=True)
    a = _mini(dt)
    b = copy.deepcopy(a)
    fuse_forward(a, attention=True)
    fuse_forward(b, attention=False)
    for L_ in (32, 64, 128):
        batch = make_batches(1, 4, 4096, seed=L_, device="cuda", fixed_len=L_)[0]
        la, lb = _loss(a, batch), _loss(b, batch)
        print(f"  L={L_}: loss {la:.6f} (library) vs {lb:.6f} (sdpa)", flush=True)
        assert abs(la - lb) <= {torch.float16: 2e-3, torch.bfloat16: 2e-2}[dt]
    # a padded batch has a mask: SDPA runs, so the two models agree bit for bit
    padded = make_batches(1, 4, 4096, seed=7, device="cuda", min_len=20, max_len=60)[0]
    assert _loss(a, padded) == _loss(b, padded)


def test_zo_run_with_library_attention_tracks_sdpa():
    """30 MeZO steps on unpadded batches at the bench's learning rate (1e-6):
    the library attention's loss trajectory stays within rounding distance of
    SDPA's. (A ZO step amplifies forward rounding: g = (L1 - L2) / 2e-3 moves
    by ~0.25 per unit in the last place of an fp16 loss near 0.7, so at a large
    learning rate any two attention kernels drift apart step by step.)"""
    import copy

    import numpy as np

    from dizo_amd.synth import make_batches
    from dizo_amd.trainer import ZOArguments, ZOTrainer

    a = _mini(torch.float16, seed=5)
    b = copy.deepcopy(a)
    batches = make_batches(30, 8, 4096, seed=4, device="cuda", fixed_len=64)
    losses = []
    for model, lib in ((a, True), (b, False)):
        np.random.seed(12)
        tr = ZOTrainer(model, ZOArguments(learning_rate=1e-6, zo_eps=1e-3, max_steps=30, zo_fused_mlp=True,
                                          zo_fused_qkv=True, zo_fused_attention=lib, zo_option_head=True))
        losses.append(torch.stack([tr.training_step(x) for x in batches]).float())
        tr.zo_flush()
        tr.zo_close()
    diff = (losses[0] - losses[1]).abs()
    print(f"[attention zo] |loss difference| over 30 steps: max {diff.max().item():.3g}, "
          f"mean {diff.mean().item():.3g}", flush=True)
    assert diff.max().item() <= 2e-3 and diff.mean().item() <= 1e-3


def test_graph_replays_library_attention_bit_identical():
    import copy

    import numpy as np

    from dizo_amd.synth import make_batches
    from dizo_amd.trainer import ZOArguments, ZOTrainer

    a = _mini(torch.float16, seed=6)
    b = copy.deepcopy(a)
    batches = make_batches(8, 4, 4096, seed=8, device="cuda", fixed_len=64)
    out = []
    for model, graph in ((a, True), (b, False)):
        np.random.seed(13)
        tr = ZOTrainer(model, ZOArguments(learning_rate=1e-3, zo_eps=1e-3, max_steps=8, zo_fused_attention=True,
                                          zo_graph=graph, zo_option_head=True))
        out.append(torch.stack([tr.training_step(x).clone() for x in batches]))
        tr.zo_flush()
        tr.zo_close()
    assert torch.equal(out[0], out[1])
    pb = dict(b.named_parameters())
    for n, p in a.named_parameters():
        assert torch.equal(p, pb[n]), n


def test_graph_with_fused_forward_across_dizo_event_bit_identical():
    """50 steps with a DiZO event (its projection table built over the k/v
    weights after they moved into the fused buffer): captured-graph steps and
    eager steps, both with the fused forward and the library attention, give
    the same losses, gamma and weights bit for bit."""
    import copy

    import numpy as np

    from dizo_amd.synth import Cycle, make_batches
    from dizo_amd.trainer import ZOArguments, ZOTrainer

    a = _mini(torch.float16, seed=7)
    b = copy.deepcopy(a)
    batches = make_batches(50, 4, 4096, seed=10, device="cuda", fixed_len=64)
    out = []
    for model, graph in ((a, True), (b, False)):
        np.random.seed(14)
        args = ZOArguments(learning_rate=1e-4, zo_eps=1e-3, max_steps=50, enhanced="zo", zo_fused_mlp=True,
                           zo_fused_qkv=True, zo_fused_attention=True, zo_graph=graph, zo_option_head=True)
        tr = ZOTrainer(model, args, train_dataloader=Cycle(batches[:6]))
        losses = torch.stack([tr.training_step(x).clone() for x in batches])
        tr.zo_flush()
        out.append((losses, tr.dizo_trainer.dizo.gamma().clone()))
        tr.zo_close()
    assert torch.equal(out[0][0], out[1][0])
    assert torch.equal(out[0][1], out[1][1])
    pb = dict(b.named_parameters())
    for n, p in a.named_parameters():
        assert torch.equal(p, pb[n]), n
