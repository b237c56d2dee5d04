"""Shared helpers of the test suite: bit-pattern conversion and input builders."""
from __future__ import annotations

import numpy as np
import torch

from oracle.arith import BF16, F16, F32, from_f32

DT_TORCH = {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}
TORCH_DT = {v: k for k, v in DT_TORCH.items()}
_INT_VIEW = {F32: torch.int32, F16: torch.int16, BF16: torch.int16}
_NP_BITS = {F32: np.uint32, F16: np.uint16, BF16: np.uint16}
_NP_SIGNED = {F32: np.int32, F16: np.int16, BF16: np.int16}


def to_torch(bits: np.ndarray, dt: str, device="cpu") -> torch.Tensor:
    arr = np.ascontiguousarray(bits.astype(_NP_BITS[dt])).view(_NP_SIGNED[dt])
    return torch.from_numpy(arr.copy()).view(DT_TORCH[dt]).to(device)


def to_bits(t: torch.Tensor) -> np.ndarray:
    dt = TORCH_DT[t.dtype]
    return t.detach().contiguous().cpu().view(_INT_VIEW[dt]).numpy().view(_NP_BITS[dt]).copy()


def edge_values(dt: str) -> np.ndarray:
    """fp32 values that exercise rounding edges of T once converted."""
    tiny = {F32: 1.4e-45, F16: 5.96e-8, BF16: 9.2e-41}[dt]
    vals = [0.0, -0.0, tiny, -tiny, 3 * tiny, 1e-30, -1e-30, 6.0e-5, -6.1e-5, 1e-3, -1e-3,
            0.02, -0.02, 1.0, -1.0, 65504.0 if dt == F16 else 1e30, 1.0000001, 3.14159]
    return np.asarray(vals, dtype=np.float32)


def random_theta(n: int, dt: str, seed: int, std: float = 0.02, with_edges: bool = True) -> np.ndarray:
    r = np.random.default_rng(seed)
    x = (r.standard_normal(n) * std).astype(np.float32)
    if with_edges and n > 64:
        e = edge_values(dt)
        idx = r.choice(n, size=min(len(e) * 4, n // 4), replace=False)
        x[idx] = np.resize(e, len(idx))
    return from_f32(x, dt)


def assert_bits_equal(got: np.ndarray, want: np.ndarray, dt: str, what: str = ""):
    """Bitwise equality, treating any two NaNs as equal."""
    g = got.astype(np.uint64)
    w = want.astype(np.uint64)
    from oracle.arith import to_f32
    gn = np.isnan(to_f32(got, dt))
    wn = np.isnan(to_f32(want, dt))
    bad = (g != w) & ~(gn & wn)
    if bad.any():
        i = np.nonzero(bad)[0][:8]
        raise AssertionError(f"{what}: {int(bad.sum())}/{len(g)} {dt} mismatches, first at {i.tolist()}: "
                             f"got {[hex(int(x)) for x in g[i]]} want {[hex(int(x)) for x in w[i]]}")
