"""CPU checks of the fused decoder-layer GEMMs (dizo_amd.fused_layers).

fc1 + ReLU: an addmm with a ReLU epilogue standing in for HF's
`activation_fn(fc1(x))` (modeling_opt.OPTDecoderLayer.forward). max(., 0)
commutes with rounding to T, so the values must equal the two-step ones bit
for bit. k/v/q: one GEMM over a [k; v; q] weight buffer standing in for
OPTAttention's three projections; on the CPU both forms run the same BLAS
routine per output column block, and the logits must not move. Under
autograd, or once the weights no longer sit side by side, HF's own code must
run, with the same values and gradients.
"""
import copy

import pytest
import torch
import torch.nn.functional as F
from transformers import OPTForCausalLM

from dizo_amd.fused_layers import FusedQKVOPTAttention, ReluLinear, fuse_forward, fuse_qkv, fuse_relu_mlp, qkv_views
from dizo_amd.synth import SHAPES, make_batches, opt_config


def _bits(t):
    return t.detach().contiguous().view({2: torch.int16, 4: torch.int32}[t.element_size()])


@pytest.fixture(scope="module")
def base():
    torch.manual_seed(11)
    return OPTForCausalLM(opt_config(SHAPES["opt-tiny"])).eval()


def _logits(model, batch):
    with torch.inference_mode():
        return model(input_ids=batch["input_ids"], attention_mask=batch["attention_mask"]).logits


def test_fuse_changes_layout_not_names(base):
    b = copy.deepcopy(base)
    names0 = [n for n, _ in b.named_parameters()]
    keys0 = list(b.state_dict().keys())
    vals0 = {k: v.clone() for k, v in b.state_dict().items()}
    got = fuse_forward(b)
    L = SHAPES["opt-tiny"].layers
    assert got == {"mlp": L, "qkv": L}
    assert [n for n, _ in b.named_parameters()] == names0
    assert list(b.state_dict().keys()) == keys0
    for k, v in b.state_dict().items():
        assert torch.equal(v, vals0[k]), k
    for layer in b.model.decoder.layers:
        assert type(layer.fc1) is ReluLinear and isinstance(layer.activation_fn, torch.nn.Identity)
        at = layer.self_attn
        assert type(at) is FusedQKVOPTAttention
        w, bias = qkv_views(at)
        d = at.embed_dim
        assert w.shape == (3 * d, d) and bias.shape == (3 * d,)
        assert torch.equal(w[:d], at.k_proj.weight) and torch.equal(w[2 * d:], at.q_proj.weight)
        assert at.v_proj.weight.data_ptr() == w.data_ptr() + d * d * w.element_size()
    assert fuse_relu_mlp(b) == 0  # already fused
    ptrs = [p.data_ptr() for p in b.parameters()]
    assert fuse_qkv(b) == L and [p.data_ptr() for p in b.parameters()] == ptrs  # layout kept


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_fused_model_logits_bit_identical(base, dt):
    a = copy.deepcopy(base).to(dt)
    b = copy.deepcopy(a)
    fuse_forward(b)
    for seed in (2, 3):
        batch = make_batches(1, 3, 512, seed=seed, device="cpu", min_len=6, max_len=17)[0]
        assert torch.equal(_bits(_logits(a, batch)), _bits(_logits(b, batch)))


def test_fallbacks_when_layout_breaks_or_autograd_records(base):
    a = copy.deepcopy(base)
    b = copy.deepcopy(a)
    fuse_forward(b)
    batch = make_batches(1, 2, 512, seed=4, device="cpu", min_len=6, max_len=12)[0]
    want = _logits(a, batch)
    # a deep copy clones each Parameter apart: the copy runs HF's attention code
    c = copy.deepcopy(b)
    assert all(qkv_views(layer.self_attn) is None for layer in c.model.decoder.layers)
    assert torch.equal(_logits(c, batch), want)
    # rebinding one weight breaks the layout of that layer only
    at = b.model.decoder.layers[0].self_attn
    at.v_proj.weight.data = at.v_proj.weight.data.clone()
    assert qkv_views(at) is None and qkv_views(b.model.decoder.layers[1].self_attn) is not None
    assert torch.equal(_logits(b, batch), want)
    # autograd: HF's code, same loss and gradients
    a.zero_grad()
    b.zero_grad()
    ids, mask = batch["input_ids"], batch["attention_mask"]
    a(input_ids=ids, attention_mask=mask).logits.float().square().mean().backward()
    b(input_ids=ids, attention_mask=mask).logits.float().square().mean().backward()
    gb = dict(b.named_parameters())
    for n, p in a.named_parameters():
        if p.grad is not None:
            assert torch.equal(p.grad, gb[n].grad), n


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1, 64), (37, 64), (5, 3, 64)])
def test_relu_linear_layer_bits(dt, shape):
    torch.manual_seed(3)
    lin = torch.nn.Linear(64, 96).to(dt)
    x = torch.randn(*shape, dtype=dt)
    want = torch.relu(F.linear(x, lin.weight, lin.bias))
    lin.__class__ = ReluLinear
    with torch.no_grad():
        got = lin(x)
    assert got.shape == want.shape and torch.equal(_bits(got), _bits(want))


def test_relu_linear_autograd_takes_two_step_path():
    torch.manual_seed(4)
    lin = torch.nn.Linear(16, 24)
    ref = copy.deepcopy(lin)
    lin.__class__ = ReluLinear
    x = torch.randn(9, 16, requires_grad=True)
    x2 = x.detach().clone().requires_grad_()
    lin(x).square().sum().backward()
    torch.relu(ref(x2)).square().sum().backward()
    assert torch.equal(x.grad, x2.grad)
    assert torch.equal(lin.weight.grad, ref.weight.grad) and torch.equal(lin.bias.grad, ref.bias.grad)
    # frozen weights and an input without grad: nothing is recorded, the fused op runs
    for p in lin.parameters():
        p.requires_grad_(False)
    assert lin(torch.randn(9, 16)).grad_fn is None


def test_models_of_other_forms_are_left_alone():
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=1,
                      num_attention_heads=2, num_key_value_heads=1)
    m = LlamaForCausalLM(cfg)
    ptrs = [p.data_ptr() for p in m.parameters()]
    assert fuse_forward(m) == {"mlp": 0, "qkv": 0}
    assert [p.data_ptr() for p in m.parameters()] == ptrs
    gelu = torch.nn.Module()
    gelu.fc1 = torch.nn.Linear(4, 4)
    gelu.activation_fn = torch.nn.GELU()
    assert fuse_relu_mlp(gelu) == 0 and type(gelu.fc1) is torch.nn.Linear
    nobias = torch.nn.Module()
    nobias.fc1 = torch.nn.Linear(4, 4, bias=False)
    nobias.activation_fn = torch.nn.ReLU()
    assert fuse_relu_mlp(nobias) == 0


def test_trainer_applies_the_fusions(base):
    from dizo_amd.trainer import ZOArguments, ZOTrainer, select_trainable

    m = copy.deepcopy(base)
    tr = ZOTrainer.__new__(ZOTrainer)
    tr.args = ZOArguments(learning_rate=1e-3, max_steps=5, enhanced=None, zo_fused_mlp=True, zo_fused_qkv=True)
    tr.zo_setup(m)  # MeZO: no table is built before the first pass
    for layer in m.model.decoder.layers:
        assert type(layer.self_attn) is FusedQKVOPTAttention and qkv_views(layer.self_attn) is not None
        assert type(layer.fc1) is ReluLinear
    assert [n for n, _ in tr.named_parameters_to_optim] == [n for n, _ in select_trainable(base)[0]]
    plain = copy.deepcopy(base)
    tr2 = ZOTrainer.__new__(ZOTrainer)
    tr2.args = ZOArguments(learning_rate=1e-3, max_steps=5, enhanced=None)
    tr2.zo_setup(plain)
    assert type(plain.model.decoder.layers[0].self_attn) is not FusedQKVOPTAttention


@pytest.mark.parametrize("enable_bias,ln_before", [(False, True), (True, False)])
def test_fusions_on_other_opt_configs(enable_bias, ln_before):
    """OPT without biases (the k/v/q buffer without a bias buffer; fc1 left as
    it is, its epilogue form needs the bias) and OPT-350m's post-norm layout:
    the same logits bit for bit."""
    from transformers import OPTConfig

    cfg = OPTConfig(vocab_size=512, hidden_size=64, num_hidden_layers=2, ffn_dim=128, num_attention_heads=4,
                    max_position_embeddings=128, word_embed_proj_dim=64, enable_bias=enable_bias,
                    do_layer_norm_before=ln_before, pad_token_id=1, dropout=0.0, attention_dropout=0.0)
    torch.manual_seed(2)
    a = OPTForCausalLM(cfg).eval()
    b = copy.deepcopy(a)
    got = fuse_forward(b)
    assert got["qkv"] == 2 and got["mlp"] == (2 if enable_bias else 0)
    w, bias = qkv_views(b.model.decoder.layers[0].self_attn)
    assert (bias is None) == (not enable_bias)
    batch = make_batches(1, 3, 512, seed=4, device="cpu", min_len=6, max_len=20)[0]
    assert torch.equal(_bits(_logits(a, batch)), _bits(_logits(b, batch)))
