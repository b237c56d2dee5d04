"""Causal attention of an unpadded batch through libdizo_amd (dz_attention_causal).

Stands in for the SDPA call of HF's OPTAttention.forward when the model
passes no mask (SDPA's is_causal path: every sequence of the batch unpadded),
in the ZO step's forwards, which run without autograd. It takes q, k and v as
the fused k/v/q GEMM leaves them (strided views of one buffer, q not yet
scaled) and applies HF's `q * scaling` itself, so the separate scaling pass
goes too.

Not bit-identical to SDPA's flash kernel (another exp and summation order);
softmax and accumulation are fp32 and P is rounded to T before the product
with V, as flash attention does. The GPU tests hold it to an fp32 reference
and compare ZO runs with SDPA's.
"""
from __future__ import annotations

import torch

from . import _lib as L
from .table import dtype_code, stream_handle

HEAD_DIMS = (64, 128)
MAX_LEN = 256


def supported(q: torch.Tensor, L_: int, head_dim: int) -> bool:
    """Shapes and dtypes the kernel takes (the caller falls back otherwise)."""
    return (q.is_cuda and q.dtype in (torch.float16, torch.bfloat16) and head_dim in HEAD_DIMS
            and 32 <= L_ <= MAX_LEN and L_ % 32 == 0)


def attention_causal(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, heads: int, head_dim: int,
                     scale: float, *, stream=None) -> torch.Tensor:
    """softmax(R_T(q * scale) k^T + causal mask) v per head, for q, k, v of shape
    (n_seq, L, heads * head_dim) whose last dim is contiguous (token and
    sequence strides free). Returns (n_seq, L, heads, head_dim), contiguous."""
    if not (q.shape == k.shape == v.shape) or q.dim() != 3:
        raise L.DzError(f"attention: q, k, v must be (n_seq, L, heads * head_dim) of one shape, got "
                        f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    n_seq, L_, width = q.shape
    if width != heads * head_dim:
        raise L.DzError(f"attention: last dim {width} != heads * head_dim = {heads * head_dim}")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != q.dtype or t.device != q.device or t.stride(2) != 1:
            raise L.DzError(f"attention: {name} must be a {q.dtype} tensor on {q.device} with a contiguous last dim")
    out = torch.empty((n_seq, L_, heads, head_dim), dtype=q.dtype, device=q.device)
    with torch.cuda.device(q.device):
        L.call("dz_attention_causal", dtype_code(q.dtype), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
               q.stride(1), k.stride(1), v.stride(1), q.stride(0), k.stride(0), v.stride(0), n_seq, L_, heads,
               head_dim, float(scale), stream_handle(stream))
    return out
