"""hipGraph capture of the zeroth-order step.

One ZO step of the reference (trainer.py:1570-1617: perturb +1, forward,
perturb -2, forward, projected_grad, restore, update) replays as one captured
graph per input shape (and padded / unpadded attention mask, since the two
take different attention paths, and option-head logit window), with no host
synchronisation:

  first  : perturb(+1, z_k) -> forward -> perturb(-2, z_k) -> forward -> g_k
  steady : restore+update(z_{k-1}, g_{k-1}, lr_{k-1}) fused with perturb(+1, z_k)
           -> forward -> perturb(-2, z_k) -> forward -> g_k

Both end with the step's restore+update pending, held as device scalars
(seed, g, lr) that the next replay's first pass or ``flush()`` consumes. The
kernels read the seed, gradient and learning rate through device pointers,
so a replay picks up the values uploaded before it; g is computed on the
device with the reference's expression ((L1 - L2) / (2 eps), trainer.py:1587)
and never read back. The model forward and the loss are captured as they run
eagerly: attention goes through an attention implementation registered here
that calls the same SDPA function with the mask HF would build eagerly (none
for an unpadded batch, so SDPA's is_causal path; HF's SDPA mask otherwise),
because HF's own mask code probes the mask on the host, which capture forbids.

A new input shape runs one eager step through the same code, then both
graphs are captured (capture records, it does not execute).
"""
from __future__ import annotations

import weakref
from typing import Dict, Optional, Tuple

import torch

from ._lib import DzError

ATTN_IMPL = "dizo_sdpa"
_state = {"unpadded": True, "registered": False}


def _mask_fn(*args, **kwargs):
    if _state["unpadded"]:
        return None
    from transformers.masking_utils import sdpa_mask

    kwargs["allow_is_causal_skip"] = False
    return sdpa_mask(*args, **kwargs)


def register_attention() -> None:
    """Registers ATTN_IMPL: HF's SDPA attention with a host-sync-free mask."""
    if _state["registered"]:
        return
    from transformers import AttentionInterface
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    from transformers.masking_utils import AttentionMaskInterface

    AttentionInterface.register(ATTN_IMPL, sdpa_attention_forward)
    AttentionMaskInterface.register(ATTN_IMPL, _mask_fn)
    _state["registered"] = True


class _Captured:
    def __init__(self):
        self.static: Dict[str, torch.Tensor] = {}
        self.nopt = None
        self.unpadded = True
        self.window = 0  # trailing positions of logits the loss reads (0: all)
        self.first: Optional[torch.cuda.CUDAGraph] = None
        self.steady: Optional[torch.cuda.CUDAGraph] = None
        self.loss1: Optional[torch.Tensor] = None  # output of `first`
        self.loss1_steady: Optional[torch.Tensor] = None  # output of `steady`


class GraphedZOStep:
    """Captured ZO steps for a ZOTrainerMixin (see the module docstring)."""

    RING = 8

    def __init__(self, trainer):
        register_attention()
        self.tr = trainer
        tabs = trainer._zo_tables()
        if len(tabs.tables) != 1:
            raise DzError("graph mode needs all ZO parameters in one dtype")
        self.tab = tabs.tables[0][0]
        self.dtype = self.tab.dtype
        dev = self.tab.device
        self.device = dev
        self.eps = float(trainer.args.zo_eps)
        self.d_cur_seed = torch.zeros(1, dtype=torch.int64, device=dev)
        self.d_prev_seed = torch.zeros(1, dtype=torch.int64, device=dev)
        self.d_cur_lr = torch.zeros(1, dtype=torch.float32, device=dev)
        self.d_prev_lr = torch.zeros(1, dtype=torch.float32, device=dev)
        self.d_prev_g = torch.zeros((), dtype=self.dtype, device=dev)
        self.h_seed = [torch.zeros(1, dtype=torch.int64).pin_memory() for _ in range(self.RING)]
        self.h_lr = [torch.zeros(1, dtype=torch.float32).pin_memory() for _ in range(self.RING)]
        self.events = [None] * self.RING
        self.slot = 0
        self.caps: Dict[Tuple, _Captured] = {}
        self.pool = None
        self.pending = False  # a restore+update waits in the d_prev_* scalars
        self.capturing = False
        self._pad_cache: Dict[int, tuple] = {}

    # ----------------------------------------------------------- body ----
    def _loss(self, cap: _Captured) -> torch.Tensor:
        from .trainer import option_len_loss

        st = cap.static
        model = self.tr.model
        model.eval()
        with torch.inference_mode():
            kw = {k: v for k, v in st.items() if k not in ("input_ids", "labels", "option_len", "num_options")}
            return option_len_loss(model, False, st["input_ids"], st.get("labels"), st.get("option_len"),
                                   cap.nopt, True, dz_window=cap.window, **kw).loss

    def _body(self, cap: _Captured, first: bool) -> torch.Tensor:
        tab, eps = self.tab, self.eps
        if first:
            tab.perturb(0, 1.0, eps, d_seed=self.d_cur_seed)
        else:
            tab.restore_update_perturb(0, 0, eps, 0.0, 0.0, d_seed=self.d_prev_seed, d_next_seed=self.d_cur_seed,
                                       d_grad=self.d_prev_g, d_lr=self.d_prev_lr)
        loss1 = self._loss(cap)
        tab.perturb(0, -2.0, eps, d_seed=self.d_cur_seed)
        loss2 = self._loss(cap)
        g = (loss1 - loss2) / (2 * eps)
        # this step's restore + update is the next replay's (or flush's) work
        self.d_prev_seed.copy_(self.d_cur_seed)
        self.d_prev_lr.copy_(self.d_cur_lr)
        self.d_prev_g.copy_(g)
        return loss1

    # ------------------------------------------------------------ host ----
    def _unpadded(self, batch) -> bool:
        """Whether every attention-mask entry is 1 (the forward then takes SDPA's
        is_causal path). Read on the host: free for a CPU batch; for a device
        batch one sync the first time that tensor is seen (cached per tensor)."""
        am = batch.get("attention_mask")
        if am is None:
            return True
        if am.device.type == "cpu":
            return bool(am.all())
        hit = self._pad_cache.get(id(am))
        if hit is not None and hit[0]() is am and hit[1] == am._version:
            return hit[2]
        flag = bool(am.all())
        self._pad_cache[id(am)] = (weakref.ref(am), am._version, flag)
        return flag

    def _window(self, batch) -> int:
        """The option head's logit window for this batch (0: full logits), decided
        on the host: capture cannot read option_len back from the device."""
        from .trainer import host_ints, option_window

        if not getattr(self.tr.model, "dz_option_head", False):
            return 0
        if any(batch.get(k) is None for k in ("labels", "option_len", "num_options")):
            return 0
        return option_window(host_ints(batch["option_len"]), batch["input_ids"].shape[1]) or 0

    def _key(self, batch) -> Tuple:
        """Graphs are reused for batches that agree in every tensor's shape and
        dtype, the option counts (they choose the loss's branch), the logit
        window and whether the mask has padding."""
        from .trainer import host_ints

        shapes = tuple((k, tuple(v.shape), v.dtype) for k, v in sorted(batch.items()) if torch.is_tensor(v))
        nopt = batch.get("num_options")
        nopt = None if nopt is None else tuple(host_ints(nopt))
        return shapes + (("nopt", nopt), ("window", self._window(batch)), ("unpadded", self._unpadded(batch)))

    def _upload(self, seed: int, lr: float) -> None:
        i = self.slot
        self.slot = (i + 1) % self.RING
        if self.events[i] is not None:
            self.events[i].synchronize()  # the pinned slot's previous copy has run
        self.h_seed[i][0] = int(seed)
        self.h_lr[i][0] = float(lr)
        self.d_cur_seed.copy_(self.h_seed[i], non_blocking=True)
        self.d_cur_lr.copy_(self.h_lr[i], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.events[i] = ev

    def _with_attention(self, cap: _Captured, fn):
        model = self.tr.model
        prev = model.config._attn_implementation
        model.config._attn_implementation = ATTN_IMPL
        _state["unpadded"] = cap.unpadded
        self.capturing = True
        try:
            return fn()
        finally:
            self.capturing = False
            model.config._attn_implementation = prev

    def _new_capture(self, batch, unpadded: bool, window: int) -> _Captured:
        from .trainer import host_ints

        cap = _Captured()
        for k, v in batch.items():
            if torch.is_tensor(v):
                cap.static[k] = v.to(self.device, copy=True)
        nopt = batch.get("num_options")
        cap.nopt = None if nopt is None else list(host_ints(nopt))
        cap.unpadded = unpadded
        cap.window = window
        return cap

    def _capture(self, cap: _Captured) -> None:
        def run():
            g1 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g1, pool=self.pool):
                cap.loss1 = self._body(cap, True)
            self.pool = g1.pool()
            g2 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g2, pool=self.pool):
                cap.loss1_steady = self._body(cap, False)
            cap.first, cap.steady = g1, g2
        # The graphs share one memory pool (also across shapes): they run one
        # at a time on one stream, and each keeps its output tensor alive.
        self._with_attention(cap, run)

    def step(self, batch, seed: int, lr: float) -> torch.Tensor:
        """One ZO step with seed `seed`; lr is the learning rate of its update
        (applied by the next step or flush). Returns loss1 (a device tensor the
        next step overwrites: clone it to keep it)."""
        self._upload(seed, lr)
        key = self._key(batch)
        cap = self.caps.get(key)
        first = not self.pending
        if cap is None:
            cap = self._new_capture(batch, key[-1][1], key[-2][1])
            # one eager step through the body (warms kernels and allocator),
            # on a side stream as capture expects
            side = torch.cuda.Stream(device=self.device)
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                loss1 = self._with_attention(cap, lambda: self._body(cap, first))
            torch.cuda.current_stream().wait_stream(side)
            self.pending = True
            loss1 = loss1.clone()
            self._capture(cap)
            self.caps[key] = cap
            return loss1
        for k, v in batch.items():
            if torch.is_tensor(v):
                cap.static[k].copy_(v, non_blocking=True)
        if first:
            cap.first.replay()
            out = cap.loss1
        else:
            cap.steady.replay()
            out = cap.loss1_steady
        self.pending = True
        return out

    def flush(self) -> None:
        """Applies the pending restore + update (eagerly, from the device scalars)."""
        if self.pending and not self.capturing:
            self.pending = False
            self.tab.restore_update(0, self.eps, 0.0, 0.0, d_seed=self.d_prev_seed, d_grad=self.d_prev_g,
                                    d_lr=self.d_prev_lr)

    def close(self) -> None:
        self.flush()
        self.caps = {}
        self.pool = None
