"""Device-side parameter tables: the torch-facing wrappers of dz_table.

A ``ZOTable`` registers the ZO-optimised tensors (``named_parameters_to_optim``,
trainer.py:1147-1160) once; perturb / update / restore+update then run as one
multi-tensor kernel each, regenerating z from (seed, element index).
A ``ProjTable`` registers the projected k/v tensors with their anchors theta0
(trainer.py:1157-1168) for the DiZO norm / apply / reverse passes.

Tables hold raw device addresses. The kernels mutate tensors in place, so
the addresses stay valid; ``check()`` raises if any storage moved (for
example after ``param.data = new_tensor``).
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import torch

from . import _lib as L
from ._lib import DzError

DTYPE_CODE = {torch.float32: L.DZ_DTYPE_F32, torch.float16: L.DZ_DTYPE_F16,
              torch.bfloat16: L.DZ_DTYPE_BF16}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise DzError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def stream_handle(stream: Optional[torch.cuda.Stream] = None) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _validate(tensors: Sequence[torch.Tensor], what: str) -> tuple[torch.device, torch.dtype]:
    if len(tensors) == 0:
        raise DzError(f"{what}: no tensors")
    dev, dt = tensors[0].device, tensors[0].dtype
    if dev.type != "cuda":
        raise DzError(f"{what}: tensors must live on a GPU, got {dev}")
    dtype_code(dt)
    for i, t in enumerate(tensors):
        if t.device != dev or t.dtype != dt:
            raise DzError(f"{what}: tensor {i} is {t.dtype} on {t.device}, expected {dt} on {dev}")
        if not t.is_contiguous():
            raise DzError(f"{what}: tensor {i} is not contiguous")
    return dev, dt


class _Table:
    def __init__(self, tensors, anchors, z_offsets, what):
        tensors = list(tensors)
        dev, dt = _validate(tensors, what)
        if anchors is not None:
            anchors = list(anchors)
            if len(anchors) != len(tensors):
                raise DzError(f"{what}: {len(anchors)} anchors for {len(tensors)} tensors")
            for i, (t, a) in enumerate(zip(tensors, anchors)):
                if a.shape != t.shape or a.dtype != t.dtype or a.device != t.device or not a.is_contiguous():
                    raise DzError(f"{what}: anchor {i} does not match its tensor "
                                  f"({tuple(a.shape)} {a.dtype} {a.device} vs {tuple(t.shape)} {t.dtype} {t.device})")
        self.device = dev
        self.dtype = dt
        self.code = dtype_code(dt)
        self.tensors = tensors
        self.anchors = anchors
        self.n = len(tensors)
        self.numels = [t.numel() for t in tensors]
        self._ptrs = [t.data_ptr() for t in tensors]
        ptrs = L.u64_array(self._ptrs)
        aptr = L.u64_array([a.data_ptr() for a in anchors]) if anchors is not None else None
        numels = L.i64_array(self.numels)
        zoffs = L.u64_array(z_offsets) if z_offsets is not None else None
        handle = C.c_void_p()
        with torch.cuda.device(dev):
            L.call("dz_table_create", ptrs, aptr, numels, zoffs, self.n, self.code,
                   dev.index, C.byref(handle))
        self._h = handle
        self.what = what

    @property
    def handle(self):
        if self._h is None:
            raise DzError(f"{self.what}: table is closed")
        return self._h

    def stale(self) -> bool:
        if any(t.data_ptr() != p for t, p in zip(self.tensors, self._ptrs)):
            return True
        return False

    def check(self) -> None:
        if self.stale():
            raise DzError(f"{self.what}: a registered tensor's storage moved since the table was "
                          "built (rebuild the table)")

    def set_prefetch_min_tiles(self, min_tiles: int) -> None:
        """Launches of the fused restore+update+next perturb pass with at least
        min_tiles tiles run the prefetching tile loop (0, the default: every
        launch; 2**32 - 1: none). The computed values do not
        depend on it."""
        L.call("dz_table_set_prefetch_min_tiles", self.handle, int(min_tiles))

    def time_next(self, start: "torch.cuda.Event | None", stop: "torch.cuda.Event | None") -> None:
        """The next launching call on this table records `start` as its first
        kernel starts and `stop` as its last kernel ends (either may be None).
        The events must have been recorded once (so that they exist)."""
        h = [None if e is None else e.cuda_event for e in (start, stop)]
        if any(x == 0 for x in h):
            raise DzError(f"{self.what}: timing events must be recorded once before time_next")
        with torch.cuda.device(self.device):
            L.call("dz_table_time_next", self.handle, h[0], h[1])

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            h, self._h = self._h, None
            with torch.cuda.device(self.device):
                L.call("dz_table_destroy", h)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ZOTable(_Table):
    """Multi-tensor ZO step over one dtype's share of the trainable set."""

    def __init__(self, tensors: Sequence[torch.Tensor], z_offsets: Optional[Sequence[int]] = None):
        super().__init__(tensors, None, z_offsets, "ZOTable")
        self.z_offsets = []
        for i in range(self.n):
            v = C.c_uint64()
            L.call("dz_table_z_offset", self.handle, i, C.byref(v))
            self.z_offsets.append(v.value)

    def perturb(self, seed: int, scale: float, eps: float, *, d_seed=None, stream=None) -> None:
        """theta <- R(theta + R(R(scale*z)*eps)) (trainer.py:1442)."""
        L.call("dz_perturb", self.handle, int(seed), float(scale), float(eps), _ptr(d_seed),
               stream_handle(stream))

    def update(self, seed: int, grad: float, lr: float, *, d_seed=None, d_grad=None, d_lr=None,
               stream=None) -> None:
        """theta <- R(theta - R(lr*R(grad*z))) (trainer.py:1608)."""
        self._check_scalar(d_grad, d_lr)
        L.call("dz_update", self.handle, int(seed), float(grad), float(lr), _ptr(d_seed),
               _ptr(d_grad), _ptr(d_lr), stream_handle(stream))

    def restore_update(self, seed: int, eps: float, grad: float, lr: float, *, d_seed=None,
                       d_grad=None, d_lr=None, stream=None) -> None:
        """Restore (+eps z, trainer.py:1593) then update (trainer.py:1608) in one pass."""
        self._check_scalar(d_grad, d_lr)
        L.call("dz_restore_update", self.handle, int(seed), float(eps), float(grad), float(lr),
               _ptr(d_seed), _ptr(d_grad), _ptr(d_lr), stream_handle(stream))

    def restore_update_perturb(self, seed: int, next_seed: int, eps: float, grad: float, lr: float, *,
                               d_seed=None, d_next_seed=None, d_grad=None, d_lr=None, stream=None) -> None:
        """Restore + update of step `seed`, then the +1 perturbation of step `next_seed`, in one pass."""
        self._check_scalar(d_grad, d_lr)
        L.call("dz_restore_update_perturb", self.handle, int(seed), int(next_seed), float(eps), float(grad),
               float(lr), _ptr(d_seed), _ptr(d_next_seed), _ptr(d_grad), _ptr(d_lr), stream_handle(stream))

    def _check_scalar(self, d_grad, d_lr):
        if d_grad is not None and (d_grad.dtype != self.dtype or d_grad.device != self.device):
            raise DzError(f"d_grad must be a {self.dtype} scalar on {self.device}")
        if d_lr is not None and (d_lr.dtype != torch.float32 or d_lr.device != self.device):
            raise DzError(f"d_lr must be a float32 scalar on {self.device}")

    def export_z(self, seed: int, idx: int, *, stream=None) -> torch.Tensor:
        """The z that perturb/update apply to tensor idx, as a tensor of its shape."""
        t = self.tensors[idx]
        out = torch.empty(t.shape, dtype=t.dtype, device=t.device)
        L.call("dz_export_z", self.handle, int(seed), int(idx), out.data_ptr(), stream_handle(stream))
        return out


class ProjTable(_Table):
    """The projected tensors (one group each) with their anchors theta0."""

    def __init__(self, tensors: Sequence[torch.Tensor], anchors: Sequence[torch.Tensor]):
        super().__init__(tensors, anchors, None, "ProjTable")
        # bytes of one read (or write) of every registered tensor
        self.bytes_per_tensor_pass = sum(n * tensors[0].element_size() for n in self.numels)

    def _outs(self, sumsq, norm_f32, norm_T):
        for name, t, dt in (("sumsq", sumsq, torch.float64), ("norm_f32", norm_f32, torch.float32),
                            ("norm_T", norm_T, self.dtype)):
            if t is not None and (t.dtype != dt or t.device != self.device or t.numel() < self.n
                                  or not t.is_contiguous()):
                raise DzError(f"{name} must be a contiguous {dt} tensor of >= {self.n} values on {self.device}")

    def group_sumsq(self, sumsq=None, norm_f32=None, norm_T=None, *, stream=None) -> None:
        """Per-group sum of squares / norm of R(theta - theta0) (trainer.py:455-457, 583)."""
        self._outs(sumsq, norm_f32, norm_T)
        L.call("dz_group_sumsq", self.handle, _ptr(sumsq), _ptr(norm_f32), _ptr(norm_T),
               stream_handle(stream))

    def project(self, alpha: torch.Tensor, mode: int, sumsq=None, norm_f32=None, norm_T=None, *,
                stream=None) -> None:
        """APPLY (trainer.py:428-436) / REVERSE (trainer.py:447-451) with per-group alpha
        (alpha in the table dtype; float32 for APPLY_F32ALPHA)."""
        want = torch.float32 if mode == L.DZ_PROJ_APPLY_F32ALPHA else self.dtype
        if alpha.dtype != want or alpha.device != self.device or alpha.numel() != self.n \
                or not alpha.is_contiguous():
            raise DzError(f"alpha must be a contiguous {want} tensor of {self.n} values on {self.device}")
        self._outs(sumsq, norm_f32, norm_T)
        L.call("dz_project", self.handle, alpha.data_ptr(), int(mode), _ptr(sumsq), _ptr(norm_f32),
               _ptr(norm_T), stream_handle(stream))


    def group_dot(self, others, dot=None, dot_f32=None, *, stream=None) -> None:
        """Per group: sum fp32(other) * fp32(R(theta - theta0)), others shaped like the tensors."""
        others = list(others)
        if len(others) != self.n:
            raise DzError(f"group_dot: {len(others)} tensors for {self.n} groups")
        for i, (o, t) in enumerate(zip(others, self.tensors)):
            if o.dtype != self.dtype or o.device != self.device or o.numel() != t.numel() or not o.is_contiguous():
                raise DzError(f"group_dot: tensor {i} must be a contiguous {self.dtype} tensor of {t.numel()} "
                              f"values on {self.device}")
        self._outs(dot, dot_f32, None)
        L.call("dz_group_dot", self.handle, L.u64_array([o.data_ptr() for o in others]), _ptr(dot),
               _ptr(dot_f32), stream_handle(stream))


def normals(seed: int, stream_id: int, offset: int, n: int, dtype: torch.dtype,
            device: torch.device, *, stream=None) -> torch.Tensor:
    """z(seed, stream_id, offset + i), i < n, as a 1-D tensor of `dtype` on `device`."""
    out = torch.empty(n, dtype=dtype, device=device)
    with torch.cuda.device(device):
        L.call("dz_normals", int(seed), int(stream_id), int(offset), int(n), dtype_code(dtype),
               out.data_ptr(), stream_handle(stream))
    return out


def philox_blocks(seed: int, stream_id: int, q0: int, n: int, device: torch.device, *,
                  stream=None) -> torch.Tensor:
    """n blocks of the z generator (Philox4x32-7) as an (n, 4) int32 tensor (bit patterns of uint32)."""
    out = torch.empty((n, 4), dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        L.call("dz_philox", int(seed), int(stream_id), int(q0), int(n), out.data_ptr(),
               stream_handle(stream))
    return out


def normal_table(dtype: torch.dtype) -> torch.Tensor:
    """The product's quantile table Q_T (host computation, no GPU)."""
    code = dtype_code(dtype)
    out = torch.empty(L.TAB_ENTRIES, dtype=dtype)
    L.call("dz_normal_table", code, out.data_ptr(), L.TAB_ENTRIES)
    return out


def philox_host(seed: int, stream_id: int, q: int) -> list[int]:
    """One block of the z generator (Philox4x32-7) computed by the library on the host."""
    out = (C.c_uint32 * 4)()
    L.call("dz_philox_host", int(seed), int(stream_id), int(q), out)
    return list(out)
