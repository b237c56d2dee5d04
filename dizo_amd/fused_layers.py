"""Faster forms of HF's OPT decoder layer for the ZO step's forwards.

The ZO step runs two forwards per step (and 20 per DiZO event) without
autograd, and at OPT-13B those forwards are ~90 % of the step. Two changes to
how the layer calls its GEMMs make them cheaper and leave every value as HF's
layer computes it on this stack; the fused attention module also gives SDPA a
padded batch's mask in additive form, made once per forward
(`_additive_mask`; the same bits).

1. fc1 + ReLU (`OPTDecoderLayer.forward`: `fc2(activation_fn(fc1(h)))`, ReLU
   for every OPT size) as one hipBLASLt call with a bias+ReLU epilogue
   (`torch._addmm_activation`): the same GEMM, with max(., 0) applied to the
   fp32 accumulator + bias before the single rounding to T. Rounding to T
   commutes with max(., 0), so the values are HF's bit for bit; the separate
   elementwise pass over the (tokens, ffn_dim) activation is gone (~55 us per
   layer at OPT-13B).

2. k/q/v projections (`OPTAttention.forward`) as one GEMM against a (3d, d)
   weight. `fuse_qkv` moves k_proj, v_proj and q_proj's weights (and biases)
   into one buffer, rows [k; v; q], and rebinds each Parameter to its rows, so
   the Parameters, their names and the ZO library's per-tensor passes are
   unchanged. The forward then splits one (tokens, 3d) output into the three
   projections. Each output element is the same dot product as before; it is
   bit-identical to the three GEMMs when hipBLASLt runs the same kernel family
   for both shapes (measured on the MI355X at OPT-2.7B and OPT-13B shapes;
   not at OPT-30B bf16, whose fused shape gets another kernel and can differ
   in the last bit). At OPT-13B it saves ~160 us per layer (623 -> 463 us).

Neither op has an autograd formula here (`_addmm_activation` has none; the
fused weight is a view the Parameters do not see), so whenever autograd would
record (the first-order gamma path, any caller training with gradients) the
layers run HF's own code. The fused attention also checks, on every call,
that the three weights still sit side by side in one buffer (a caller may
rebind `param.data`, or `copy.deepcopy` may clone each Parameter apart) and
runs HF's code when they do not.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F
from torch import nn
from transformers.models.opt import modeling_opt as _opt


def _records(x: torch.Tensor, *params) -> bool:
    """True when autograd would record an op on x and these parameters."""
    if not torch.is_grad_enabled():
        return False
    return x.requires_grad or any(p is not None and p.requires_grad for p in params)


class ReluLinear(nn.Linear):
    """nn.Linear followed by ReLU, fused into the GEMM when nothing is recorded."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if _records(x, self.weight, self.bias):
            return torch.relu(F.linear(x, self.weight, self.bias))
        x2 = x.reshape(-1, x.shape[-1])
        y = torch._addmm_activation(self.bias, x2, self.weight.t(), use_gelu=False)
        return y.view(*x.shape[:-1], y.shape[-1])


def _is_relu(m) -> bool:
    return isinstance(m, nn.ReLU)


def fuse_relu_mlp(model: nn.Module) -> int:
    """Turns every layer with `fc1` (a biased nn.Linear) followed by a ReLU
    `activation_fn` (HF OPT's decoder layer) into the fused form, in place.
    Returns the number of layers changed; layers of another form (LLaMA's
    gated SiLU MLP, a GELU MLP) are left as they are. A second call changes
    nothing."""
    n = 0
    for mod in model.modules():
        fc1 = getattr(mod, "fc1", None)
        act = getattr(mod, "activation_fn", None)
        if type(fc1) is nn.Linear and fc1.bias is not None and act is not None and _is_relu(act):
            fc1.__class__ = ReluLinear
            mod.activation_fn = nn.Identity()
            n += 1
    return n


def _adjacent_rows(ts) -> Optional[torch.Tensor]:
    """The (sum of rows, ...) view over tensors that lie one after another in
    one storage, in this order, each contiguous; None otherwise."""
    first = ts[0]
    if any(not t.is_contiguous() or t.dtype != first.dtype or t.device != first.device
           or t.shape[1:] != first.shape[1:] for t in ts):
        return None
    es = first.element_size()
    ptr = first.data_ptr()
    for t in ts:
        if t.data_ptr() != ptr:
            return None
        ptr += t.numel() * es
    storage = first.untyped_storage()
    if ptr > storage.data_ptr() + storage.nbytes():
        return None
    rows = sum(t.shape[0] for t in ts)
    shape = (rows, *first.shape[1:])
    return first.as_strided(shape, first.stride(), first.storage_offset())


def qkv_views(attn) -> Optional[tuple]:
    """(weight, bias) views of the fused [k; v; q] buffers of an attention
    module, or None if its three projections are not (or no longer) laid out
    that way. bias is None when the projections have none."""
    k, v, q = attn.k_proj, attn.v_proj, attn.q_proj
    w = _adjacent_rows([k.weight, v.weight, q.weight])
    if w is None:
        return None
    if k.bias is None and v.bias is None and q.bias is None:
        return w, None
    if k.bias is None or v.bias is None or q.bias is None:
        return None
    b = _adjacent_rows([k.bias, v.bias, q.bias])
    return None if b is None else (w, b)


# attention implementations whose `attention_mask is None` means causal (SDPA's
# is_causal path): HF's SDPA and the capture-safe registration in dizo_amd.graph
_SDPA_IMPLS = ("sdpa", "dizo_sdpa")

# (mask, dtype, additive form) of the last boolean mask converted
_mask_cache: list = [None, None, None]


def _additive_mask(mask: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """SDPA's additive form of a boolean mask (0 where attended, -inf
    elsewhere), made once per mask object: HF passes one mask tensor to every
    layer of a forward, and SDPA given the boolean one converts it on every
    call (two fills and a select per layer). SDPA gives the same bits with
    either form."""
    if _mask_cache[0] is mask and _mask_cache[1] == dtype:
        return _mask_cache[2]
    add = torch.zeros(mask.shape, dtype=dtype, device=mask.device).masked_fill_(~mask, float("-inf"))
    _mask_cache[:] = [mask, dtype, add]
    return add


class FusedQKVOPTAttention(_opt.OPTAttention):
    """OPTAttention whose three input projections run as one GEMM (module doc)."""

    def forward(self, hidden_states: torch.Tensor, past_key_values=None, attention_mask=None,
                output_attentions: bool = False, **kwargs):
        fused = None
        if past_key_values is None and not _records(
                hidden_states, self.k_proj.weight, self.v_proj.weight, self.q_proj.weight,
                self.k_proj.bias, self.v_proj.bias, self.q_proj.bias):
            fused = qkv_views(self)
        if fused is None:
            return super().forward(hidden_states, past_key_values=past_key_values, attention_mask=attention_mask,
                                   output_attentions=output_attentions, **kwargs)
        w, b = fused
        bsz, tgt_len, _ = hidden_states.size()
        k, v, q = F.linear(hidden_states, w, b).split(self.embed_dim, dim=-1)
        if (attention_mask is not None and attention_mask.dtype == torch.bool
                and self.config._attn_implementation in _SDPA_IMPLS):
            attention_mask = _additive_mask(attention_mask, q.dtype)
        # HF's order: q rounded to T by the GEMM, then scaled (one more rounding)
        query_states = (q * self.scaling).view(bsz, -1, self.num_heads, self.head_dim).transpose(1, 2)
        key_states = k.view(bsz, -1, self.num_heads, self.head_dim).transpose(1, 2)
        value_states = v.view(bsz, -1, self.num_heads, self.head_dim).transpose(1, 2)
        attention_interface = _opt.ALL_ATTENTION_FUNCTIONS.get_interface(
            self.config._attn_implementation, _opt.eager_attention_forward)
        attn_output, attn_weights = attention_interface(
            self, query_states, key_states, value_states, attention_mask,
            dropout=0.0 if not self.training else self.dropout, scaling=1.0, **kwargs)
        attn_output = attn_output.reshape(bsz, tgt_len, -1).contiguous()
        return self.out_proj(attn_output), attn_weights


def fuse_qkv(model: nn.Module) -> int:
    """Lays every OPT attention's k/v/q projection weights (and biases) out as
    one [k; v; q] buffer and switches the module to the fused forward, in
    place. Call it before anything records the parameters' addresses (the ZO
    trainer does it before building its tables). Returns the number of
    attention modules fused; a second call changes nothing."""
    n = 0
    for mod in model.modules():
        if not isinstance(mod, _opt.OPTAttention):
            continue
        k, v, q = mod.k_proj, mod.v_proj, mod.q_proj
        if not (k.weight.shape == v.weight.shape == q.weight.shape) or \
                len({k.weight.dtype, v.weight.dtype, q.weight.dtype}) != 1:
            continue
        if qkv_views(mod) is None:
            with torch.no_grad():
                w = torch.cat([k.weight, v.weight, q.weight], 0)
                rows = k.weight.shape[0]
                k.weight.data, v.weight.data, q.weight.data = w[:rows], w[rows:2 * rows], w[2 * rows:]
                if k.bias is not None and v.bias is not None and q.bias is not None:
                    b = torch.cat([k.bias, v.bias, q.bias], 0)
                    k.bias.data, v.bias.data, q.bias.data = b[:rows], b[rows:2 * rows], b[2 * rows:]
            if qkv_views(mod) is None:
                continue
        if type(mod) is _opt.OPTAttention:
            mod.__class__ = FusedQKVOPTAttention
        n += 1
    return n


def fuse_forward(model: nn.Module, mlp: bool = True, qkv: bool = True) -> dict:
    """The fusions asked for; returns how many layers each changed."""
    return {"mlp": fuse_relu_mlp(model) if mlp else 0, "qkv": fuse_qkv(model) if qkv else 0}
