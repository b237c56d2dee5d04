"""Drop-in zeroth-order (MeZO) step of the reference trainer, on the HIP kernels.

``ZOTrainerMixin`` carries the reference's ZO surface with unchanged
signatures and attributes (luozoupi/DiZO, large_models/trainer.py):

  zo_perturb_parameters(random_seed=None, scaling_factor=1)   trainer.py:1429-1444
  forward_wrap_with_option_len(model, input_ids, ...)         trainer.py:1446-1522
  zo_forward(model, inputs)                                   trainer.py:1524-1542
  zo_step(model, inputs)                                      trainer.py:1570-1595
  zo_update(args, model)                                      trainer.py:1597-1617

plus ``zo_setup`` for the per-run set-up the reference does inside its training
loop (ZO LambdaLR, trainer.py:1099-1101; trainable set, exclude list and the
DiZO anchor, trainer.py:1147-1171). It can be mixed into a
``transformers.Trainer`` subclass exactly where the reference defines these
methods; ``ZOTrainer`` is a self-contained host that keeps the reference's
per-step contract (trainer.py:1206-1326) without the HF Trainer machinery.

What differs from the reference, by design:
  * z is never materialised: every pass regenerates it from (seed, element
    index) inside the kernel, so ``random_vector`` (trainer.py:1444) stays
    empty (``export_z`` returns a tensor's z on demand);
  * parameters are updated in place (the reference rebinds ``param.data``),
    so the device tables of parameter addresses stay valid; a rebinding by
    user code is detected and the tables are rebuilt;
  * the restore pass that ends ``zo_step`` is deferred and fused with the
    update pass of ``zo_update`` (one read-modify-write instead of two, with
    the same per-element arithmetic); with ``zo_fuse_next_perturb`` that pass
    is deferred again and fused with the first perturbation of the next
    ``zo_step`` (two passes per step instead of three). Any forward of the
    model, any other perturbation and ``zo_flush()`` apply pending work
    first, so the parameters a caller can observe through the model are the
    reference's (code that reads parameter storage directly between two steps
    calls ``zo_flush()`` first);
  * ``torch.normal`` z (torch's Philox + Box-Muller) is replaced by the
    library's z: Philox4x32-7 keyed by the seed, 16 bits per element mapped
    through a 15-bit normal quantile table. Seeds, scaling factors, rounding
    and the update formula are the reference's.
"""
from __future__ import annotations

import json
import signal
import warnings
import weakref
from collections import OrderedDict
from dataclasses import dataclass
from types import SimpleNamespace
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch
import torch.nn.functional as F
from torch.nn import CrossEntropyLoss

from ._lib import DzError
from .table import ZOTable

EMBED_TOKENS = "model.decoder.embed_tokens.weight"
PROJECTED_SUFFIXES = ("self_attn.k_proj.weight", "self_attn.v_proj.weight")
DIZO_INTERVAL = 50  # trainer.py:1611


@dataclass
class ZOArguments:
    """The fields of the reference's OurArguments / TrainingArguments that the
    ZO step reads (run.py:35-118; defaults of dizo.sh where it sets them)."""

    learning_rate: float = 1e-7
    zo_eps: float = 1e-3
    max_steps: int = 20000
    enhanced: Optional[str] = None  # None | "zo" | "fo" (dizo.sh passes the string "None"); build: "grid"
    gradient_accumulation_steps: int = 1
    non_diff: bool = False
    n_gpu: int = 1
    logging_nan_inf_filter: bool = True
    seed: int = 26
    # build-specific pass fusion (same per-element arithmetic, fewer passes):
    # the restore of zo_step with the update of zo_update, and that pass with
    # the first perturbation of the next zo_step
    zo_fuse_restore: bool = True
    zo_fuse_next_perturb: bool = True
    # build-specific: read projected_grad back to the host in every zo_step,
    # as trainer.py:1587 does (.item()). By default the quotient stays on the
    # device, the kernels read it there, and the host reads it only when the
    # attribute is asked for: the step then has no synchronisation and the
    # next pass queues behind the second forward (same values bit for bit)
    zo_host_grad: bool = False
    # build-specific: replay each step as a captured hipGraph (ZOTrainer only)
    zo_graph: bool = False
    # build-specific: compute logits only at the option positions the
    # classification loss reads (HF's logits_to_keep) instead of at every
    # position; the loss agrees with the full-logit one to rounding
    zo_option_head: bool = False
    # build-specific: run each OPT decoder layer's fc1 + ReLU as one GEMM with
    # a ReLU epilogue, and its k/v/q projections as one GEMM over a [k; v; q]
    # weight buffer, when no autograd graph is recorded (dizo_amd.fused_layers);
    # the same values where hipBLASLt runs one kernel family for both shapes
    zo_fused_mlp: bool = False
    zo_fused_qkv: bool = False
    # build-specific: keep a journal of every pass that changes the trainable
    # tensors (seed, g, lr per step; DiZO projections), for exact replay and
    # checkpoints (dizo_amd.checkpoint)
    zo_journal: bool = False
    # build-specific: ratios tried by ENHANCED=grid (the searched-ratio DiZO
    # event: loss at each ratio, best applied); None = 8 values in [0.5, 1.0]
    dizo_grid: Optional[Tuple[float, ...]] = None
    # build-specific: append one JSON line per step (step, seed, loss1, loss2,
    # projected_grad, lr) to this file, written every 50 steps and at the end
    # (the values stay on the device until then: no extra synchronisation)
    zo_log_path: Optional[str] = None


def layout_z_offsets(numels: Sequence[int]) -> List[int]:
    """Global z index of each tensor's first element: tensors laid end to end in
    named_parameters_to_optim order, each rounded up to 8 elements."""
    offs, z = [], 0
    for n in numels:
        offs.append(z)
        z += (int(n) + 7) // 8 * 8
    return offs


def select_trainable(model: torch.nn.Module) -> Tuple[List[Tuple[str, torch.nn.Parameter]], List[str]]:
    """named_parameters_to_optim and exclude_list as trainer.py:1147-1160 builds them.

    The ZO set is every parameter with requires_grad, minus the token
    embedding when it comes first (OPT); the projected (DiZO) set is the
    k_proj / v_proj weights; everything else is in exclude_list.
    """
    named = [(n, p) for n, p in model.named_parameters() if p.requires_grad]
    if not named:
        raise DzError("model has no parameters with requires_grad")
    if named[0][0] != EMBED_TOKENS:
        exclude = [k for k in model.state_dict().keys() if "lora" not in k]
    else:
        exclude = [EMBED_TOKENS] + [n for n, _ in named if not n.endswith(PROJECTED_SUFFIXES)]
        named = named[1:]
    return named, exclude


_HOST_INTS: "OrderedDict[int, tuple]" = OrderedDict()
_HOST_INTS_MAX = 256


def host_ints(x) -> List[int]:
    """The integers of a small per-batch field (option_len, num_options) on the
    host. A list or a CPU tensor is read directly; a device tensor is copied
    back once and remembered by identity and version, so a batch that is used
    for both forwards of a step (or again in later steps) costs one copy."""
    if not torch.is_tensor(x):
        return [int(v) for v in x]
    if x.device.type == "cpu":
        return [int(v) for v in x.tolist()]
    try:
        version = x._version
    except RuntimeError:  # inference tensors carry no version counter
        return [int(v) for v in x.tolist()]
    hit = _HOST_INTS.get(id(x))
    if hit is not None and hit[0]() is x and hit[1] == version:
        return hit[2]
    vals = [int(v) for v in x.tolist()]
    _HOST_INTS[id(x)] = (weakref.ref(x), version, vals)
    if len(_HOST_INTS) > _HOST_INTS_MAX:
        _HOST_INTS.popitem(last=False)
    return vals


def option_window(option_len: Sequence[int], seq_len: int) -> Optional[int]:
    """How many trailing positions of logits the option-masked loss reads:
    max(option_len) + 1 (the logits at position j predict token j + 1). None
    when that is the whole sequence, or when some option_len is 0: the
    reference's ``shift_labels[i, :-0]`` is an empty slice, so such a row
    keeps every position (trainer.py:1473-1475)."""
    if len(option_len) == 0 or min(option_len) <= 0:
        return None
    k = max(option_len) + 1
    return k if k < seq_len else None


def shift_option_labels(input_ids: torch.Tensor, option_len, pad_id: int,
                        window: Optional[int] = None) -> torch.Tensor:
    """trainer.py:1469-1475: next-token targets, -100 at pad ids and at every
    position before each row's last option_len tokens. Over all L - 1 shifted
    positions, or over the last window - 1 of them when window is given.

    The reference's per-row loop ``shift_labels[i, :-len] = -100`` is written as
    one mask that sets the same elements: shifted position p is masked when
    p < (L - 1) - len and len > 0 (the slice [:-0] is empty). masked_fill_
    needs no device-to-host sync, so the loss can be captured in a graph."""
    L = input_ids.shape[1]
    first = 1 if window is None else L - window + 1  # first target position
    labels = torch.clone(input_ids)[..., first:].contiguous()
    if pad_id is not None:  # a config without a pad id (LLaMA) masks nothing, as `labels == None` does
        labels.masked_fill_(labels == pad_id, -100)
    if option_len is not None:
        ol = torch.as_tensor(option_len, device=labels.device).reshape(-1, 1)
        pos = torch.arange(first - 1, L - 1, device=labels.device).reshape(1, -1)
        labels.masked_fill_((pos < (L - 1) - ol) & (ol > 0), -100)
    return labels


def option_len_loss(model, build_graph: bool, input_ids=None, labels=None, option_len=None, num_options=None,
                    return_dict=None, *, dz_window: Optional[int] = None, **kwargs):
    """The option-masked classification loss of trainer.py:1446-1522 (and of its
    copy in DiZO, trainer.py:470-542, which differs only by building the
    autograd graph: build_graph=True).

    Same torch operations in the same order, so the loss (in the model dtype)
    is the reference's for the same logits. The forward runs without a
    key/value cache (use_cache=False unless the caller says otherwise): a loss
    never reads it, and building it costs two concatenations per layer; the
    logits are the same.

    Option head (``model.dz_option_head``, or an explicit ``dz_window``): the
    classification branch reads the logits of the last max(option_len) + 1
    positions only, so the forward asks HF for just those (logits_to_keep)
    and the LM head, log_softmax and gather run over that window; the masked
    positions outside it contribute nothing in the reference. The per-row
    arithmetic is the same; the LM-head GEMM has fewer rows, so the logits,
    and with them the loss, can differ from the full-logit ones by rounding.
    With the option head and return_dict falsy the logits returned are the
    window's. dz_window = 0 asks for the full logits without looking at
    option_len (a captured graph decides the window on the host beforehand).
    """
    kwargs.setdefault("use_cache", False)
    window = dz_window
    if (window is None and labels is not None and option_len is not None and num_options is not None
            and getattr(model, "dz_option_head", False)):
        window = option_window(host_ints(option_len), input_ids.shape[1])
    window = window or None
    if window is not None:
        # as index positions, not a count: HF then gathers the window's hidden
        # states into a contiguous tensor; the strided slice a count gives
        # sends the LM-head GEMM to a ~20x slower kernel once the weights stop
        # requiring grad (the DiZO projection clears requires_grad on every
        # parameter, trainer.py:417)
        L = input_ids.shape[1]
        kwargs["logits_to_keep"] = torch.arange(L - window, L, device=input_ids.device)
    if build_graph:
        outputs = model.forward(input_ids=input_ids, **kwargs)
    else:
        with torch.no_grad():
            outputs = model.forward(input_ids=input_ids, **kwargs)
    if labels is None:
        return outputs
    logits = outputs.logits
    shift_logits = logits[..., :-1, :].contiguous()
    shift_labels = shift_option_labels(input_ids, option_len, model.config.pad_token_id, window)
    loss_fct = CrossEntropyLoss(ignore_index=-100)
    if num_options is not None:
        log_probs = F.log_softmax(shift_logits, dim=-1)
        mask = shift_labels != -100
        shift_labels.masked_fill_(~mask, 0)
        selected = torch.gather(log_probs, dim=-1, index=shift_labels.unsqueeze(-1)).squeeze(-1)
        selected = (selected * mask).sum(-1) / mask.sum(-1)
        nopt = host_ints(num_options)
        if any(x != nopt[0] for x in nopt):
            loss, start, count = 0, 0, 0
            while start < len(nopt):
                end = start + nopt[start]
                loss = loss_fct(selected[start:end].unsqueeze(0), labels[start:end][0].unsqueeze(0)) + loss
                count += 1
                start = end
            loss = loss / count
        else:
            selected = selected.view(-1, nopt[0])
            loss = loss_fct(selected, labels.view(-1, nopt[0])[:, 0])
    else:
        loss = loss_fct(shift_logits.view(-1, model.config.vocab_size), shift_labels.view(-1))
    if not return_dict:
        return (loss, logits) + tuple(outputs[1:])
    return SimpleNamespace(loss=loss)


def forward_wrap_with_option_len(self, input_ids=None, labels=None, option_len=None, num_options=None,
                                 return_dict=None, **kwargs):
    """trainer.py:1446-1522 (``self`` is the model): the ZO forward's loss, no autograd graph."""
    return option_len_loss(self, False, input_ids, labels, option_len, num_options, return_dict, **kwargs)


class _ZOTables:
    """One ZOTable per dtype present in named_parameters_to_optim, sharing one
    global z layout (so z does not depend on how dtypes are grouped)."""

    def __init__(self, named: Sequence[Tuple[str, torch.nn.Parameter]]):
        self.names = [n for n, _ in named]
        self.params = [p for _, p in named]
        self.z_offsets = layout_z_offsets([p.numel() for p in self.params])
        self._ptrs = [p.data_ptr() for p in self.params]
        groups: Dict[torch.dtype, List[int]] = {}
        for i, p in enumerate(self.params):
            groups.setdefault(p.dtype, []).append(i)
        self.tables: List[Tuple[ZOTable, List[int]]] = []
        for idx in groups.values():
            tab = ZOTable([self.params[i].data for i in idx], z_offsets=[self.z_offsets[i] for i in idx])
            self.tables.append((tab, idx))
        self.bytes_per_pass = sum(2 * p.numel() * p.element_size() for p in self.params)

    def stale(self) -> bool:
        return any(p.data_ptr() != q for p, q in zip(self.params, self._ptrs))

    def close(self):
        for tab, _ in self.tables:
            tab.close()
        self.tables = []


def _grad_args(g):
    """(value, device scalar) arguments of a table call for a projected
    gradient held as a float or as a device scalar of the table's dtype."""
    return (0.0, g) if torch.is_tensor(g) else (float(g), None)


class ZOTrainerMixin:
    """The reference's ZO step methods, running on the library's kernels.

    Expects ``self.args`` (ZOArguments fields), ``self.state.global_step``,
    ``self.lr_scheduler`` and ``self._get_learning_rate()`` as on an HF
    Trainer; ``zo_setup`` provides all of them when absent.
    """

    forward_wrap_with_option_len = staticmethod(forward_wrap_with_option_len)

    # ------------------------------------------------------------ set-up --
    def zo_setup(self, model: torch.nn.Module, train_dataloader=None, *, base_model=None,
                 optimizer: Optional[torch.optim.Optimizer] = None) -> None:
        """trainer.py:1099-1101 (ZO LambdaLR) and trainer.py:1147-1171 (trainable
        set, exclude list, DiZO anchor and driver)."""
        from .dizo import dizo_trainer

        args = self.args
        self.model = model
        if not hasattr(self, "state"):
            self.state = SimpleNamespace(global_step=0)
        if optimizer is None:
            # the ZO path reads only the learning rate of the optimizer's group
            optimizer = torch.optim.SGD([torch.zeros(1, requires_grad=True)], lr=args.learning_rate)
        self.optimizer = optimizer
        # the ZO path steps the scheduler without optimizer.step(), as the reference does
        warnings.filterwarnings("ignore", message=r"Detected call of `lr_scheduler.step\(\)` before")
        self.lr_scheduler = torch.optim.lr_scheduler.LambdaLR(
            optimizer, lambda step: 1 - self.state.global_step / (2 * args.max_steps))
        self.named_parameters_to_optim, self.exclude_list = select_trainable(model)
        enhanced = args.enhanced in ("zo", "fo", "grid")
        if enhanced and base_model is None:
            base_model = _anchor_copy(model, self.exclude_list)
        # the fused q/k/v layout moves those weights into new buffers: after the
        # anchor copy, before any table records parameter addresses
        if getattr(args, "zo_fused_mlp", False) or getattr(args, "zo_fused_qkv", False):
            from .fused_layers import fuse_forward

            fuse_forward(model, mlp=bool(getattr(args, "zo_fused_mlp", False)),
                         qkv=bool(getattr(args, "zo_fused_qkv", False)))
        if enhanced:
            self.base_model = base_model
            self.dizo_trainer = dizo_trainer(base_model, train_dataloader, "l2norm", 0.1, 10, self.exclude_list)
            self.dizo_trainer.bind_model(model)
        else:
            args.enhanced = None
        self.loss_list = []
        self.random_vector = {}
        self.zo_random_seed = None
        self.projected_grad = None
        self._zo_tabs = None
        self._pending_restore = None  # (seed, eps): the +1 that ends zo_step
        self._pending_update = None   # (seed, eps, g, lr): restore + update of zo_update
        self.kernel_timer = None
        model.dz_option_head = bool(getattr(args, "zo_option_head", False))
        self.zo_journal = None
        if getattr(args, "zo_journal", False):
            from .checkpoint import ZOJournal

            projected = self.dizo_trainer.dizo.constraints_name if args.enhanced else []
            self.zo_journal = ZOJournal.for_params(self.named_parameters_to_optim, args.zo_eps, projected)
            if args.enhanced:
                self.dizo_trainer.dizo.journal = self.zo_journal
        self._hook = model.register_forward_pre_hook(lambda m, a: self.zo_flush())

    def _get_learning_rate(self) -> float:
        return self.lr_scheduler.get_last_lr()[0]

    @property
    def projected_grad(self):
        """trainer.py:1587: ((loss1 - loss2) / (2 * zo_eps)).item(), a Python
        float. zo_step may keep the quotient as a device scalar (see
        ZOArguments.zo_host_grad); reading the attribute then synchronises
        once and keeps the float."""
        g = self.__dict__.get("_projected_grad")
        if torch.is_tensor(g):
            g = float(g.item())
            self.__dict__["_projected_grad"] = g
        return g

    @projected_grad.setter
    def projected_grad(self, value) -> None:
        self.__dict__["_projected_grad"] = value

    def _grad_value(self):
        """The projected gradient as zo_step left it: a float, or a device
        scalar of the ZO tables' dtype that the kernels read in place."""
        return self.__dict__.get("_projected_grad")

    def _device_grad_ok(self, g: torch.Tensor) -> bool:
        """Whether the kernels can read g where it is: one element of every ZO
        table's dtype, on their device. The reference's g is the loss's value
        (a value of the loss dtype), and the kernels read a device g as a value
        of T, so this holds exactly when the loss dtype is T."""
        if getattr(self.args, "zo_host_grad", False) or g.numel() != 1:
            return False
        return all(t.dtype == g.dtype and t.device == g.device for t, _ in self._zo_tables().tables)

    def _zo_tables(self) -> _ZOTables:
        tabs = self._zo_tabs
        if tabs is None or tabs.stale():
            if tabs is not None:
                tabs.close()
            tabs = self._zo_tabs = _ZOTables(self.named_parameters_to_optim)
        return tabs

    def _launch(self, what: str, fn, tabs: _ZOTables) -> None:
        timer = self.kernel_timer
        if timer is None:
            for tab, _ in tabs.tables:
                fn(tab)
        else:
            with timer.span(what, tabs.bytes_per_pass, [tab for tab, _ in tabs.tables]):
                for tab, _ in tabs.tables:
                    fn(tab)

    # -------------------------------------------------------------- step --
    def zo_flush(self) -> None:
        """Applies deferred work: a pending restore+update, or a pending restore
        (the +1 perturbation that ends zo_step)."""
        graph = getattr(self, "_graph", None)
        if graph is not None:
            if graph.capturing:
                return  # the captured step manages the parameters itself
            graph.flush()
        pu = self._pending_update
        if pu is not None:
            self._pending_update = None
            seed, eps, g, lr = pu
            gv, gd = _grad_args(g)
            tabs = self._zo_tables()
            self._launch("restore_update", lambda t: t.restore_update(seed, eps, gv, lr, d_grad=gd), tabs)
        pending = self._pending_restore
        if pending is not None:
            self._pending_restore = None
            seed, eps = pending
            tabs = self._zo_tables()
            self._launch("perturb", lambda t: t.perturb(seed, 1.0, eps), tabs)

    def zo_perturb_parameters(self, random_seed=None, scaling_factor=1):
        """trainer.py:1429-1444: theta <- theta + scaling_factor * z * zo_eps, in place."""
        seed = random_seed if random_seed is not None else self.zo_random_seed
        eps = float(self.args.zo_eps)
        s = float(scaling_factor)
        pu = self._pending_update
        if pu is not None and s == 1.0 and pu[1] == eps and self._pending_restore is None:
            # previous step's restore + update, then this +1, in one pass
            self._pending_update = None
            tabs = self._zo_tables()
            prev, _, g, lr = pu
            gv, gd = _grad_args(g)
            self._launch("restore_update_perturb",
                         lambda t: t.restore_update_perturb(prev, seed, eps, gv, lr, d_grad=gd), tabs)
            # the reference re-seeds torch's generators here; the kernels do not
            # use them, so the launch goes first
            torch.manual_seed(seed)
            return
        self.zo_flush()
        tabs = self._zo_tables()
        self._launch("perturb", lambda t: t.perturb(seed, s, eps), tabs)
        torch.manual_seed(seed)  # the reference re-seeds torch's generators here

    def _prepare_inputs(self, inputs):
        dev = self.named_parameters_to_optim[0][1].device
        return {k: (v.to(dev, non_blocking=True) if torch.is_tensor(v) else v) for k, v in inputs.items()}

    def zo_forward(self, model, inputs):
        """trainer.py:1524-1542."""
        model.eval()
        if getattr(self.args, "non_diff", False):
            raise NotImplementedError("the non-differentiable (SQuAD F1) objective is not part of this library")
        with torch.inference_mode():
            inputs = self._prepare_inputs(inputs)
            loss = self.forward_wrap_with_option_len(model, **inputs, return_dict=True).loss
            if getattr(self.args, "n_gpu", 1) > 1:
                loss = loss.mean()
        return loss.detach()

    def zo_step(self, model, inputs):
        """trainer.py:1570-1595. Returns loss1; sets zo_random_seed and projected_grad."""
        args = self.args
        self.zo_random_seed = np.random.randint(1000000000)
        self.zo_perturb_parameters(scaling_factor=1)
        loss1 = self.zo_forward(model, inputs)
        self.zo_perturb_parameters(scaling_factor=-2)
        loss2 = self.zo_forward(model, inputs)
        self._last_loss2 = loss2
        g = (loss1 - loss2) / (2 * self.args.zo_eps)
        # trainer.py:1587 reads g back here (.item()); kept on the device, the
        # host does not wait for the second forward (see projected_grad)
        self.projected_grad = g if self._device_grad_ok(g) else g.item()
        assert self.args.gradient_accumulation_steps == 1
        if getattr(args, "zo_fuse_restore", True):
            self._pending_restore = (self.zo_random_seed, float(args.zo_eps))
        else:
            self.zo_perturb_parameters(scaling_factor=1)
        return loss1

    def zo_update(self, args, model):
        """trainer.py:1597-1617: theta <- theta - lr * (projected_grad * z), the
        DiZO event every 50 steps, then the scheduler step."""
        seed = self.zo_random_seed
        torch.manual_seed(seed)
        g, lr = self._grad_value(), float(self._get_learning_rate())
        gv, gd = _grad_args(g)
        event_due = (self.state.global_step + 1) % DIZO_INTERVAL == 0 and args.enhanced
        pending = self._pending_restore
        if pending is not None and pending[0] == seed:
            self._pending_restore = None
            eps = pending[1]
            if getattr(args, "zo_fuse_next_perturb", False) and not event_due:
                self._pending_update = (seed, eps, g, lr)  # applied with the next +1 perturbation
            else:
                self._launch("restore_update", lambda t: t.restore_update(seed, eps, gv, lr, d_grad=gd),
                             self._zo_tables())
        else:
            self.zo_flush()
            self._launch("update", lambda t: t.update(seed, gv, lr, d_grad=gd), self._zo_tables())
        if self.zo_journal is not None:
            self.zo_journal.zo(seed, g, lr)
        if event_due:
            self._dizo_event(model, seed)
        self.lr_scheduler.step()

    def _dizo_event(self, model, seed: int) -> None:
        """The DiZO event of trainer.py:1611-1615 (after the update of every 50th step)."""
        args = self.args
        self.zo_flush()
        self.dizo_trainer.gamma_seed = seed
        if args.enhanced == "zo":
            self.dizo_trainer.dizo_zo_iters(model, base_model=self.base_model)
        elif args.enhanced == "fo":
            self.dizo_trainer.dizo_iters(model, base_model=self.base_model)
        else:
            grid = args.dizo_grid if args.dizo_grid is not None else tuple(np.linspace(0.5, 1.0, 8))
            self.dizo_trainer.dizo_grid_iters(model, self.base_model, grid)

    def export_z(self, name: str, seed: Optional[int] = None) -> torch.Tensor:
        """The z that seed (default: the current zo_random_seed) applies to
        parameter `name` (what the reference would hold in random_vector[name])."""
        tabs = self._zo_tables()
        i = tabs.names.index(name)
        seed = self.zo_random_seed if seed is None else seed
        for tab, idx in tabs.tables:
            if i in idx:
                return tab.export_z(int(seed), idx.index(i))
        raise KeyError(name)

    def zo_close(self) -> None:
        self.zo_flush()
        if hasattr(self, "flush_log"):
            self.flush_log()
        if getattr(self, "_graph", None) is not None:
            self._graph.close()
            self._graph = None
        if self._zo_tabs is not None:
            self._zo_tabs.close()
            self._zo_tabs = None
        if getattr(self, "dizo_trainer", None) is not None:
            self.dizo_trainer.close()
        if getattr(self, "_hook", None) is not None:
            self._hook.remove()
            self._hook = None


def _anchor_copy(model: torch.nn.Module, exclude_list: Sequence[str]) -> torch.nn.Module:
    """theta0 as the reference keeps it (trainer.py:1163-1167): a copy of the
    model whose excluded (non-projected) tensors live on the CPU. Only the
    projected tensors are copied on the device here; the rest are CPU copies."""
    import copy

    excl = set(exclude_list)
    memo = {}
    for name, p in model.named_parameters():
        if name in excl:
            memo[id(p)] = torch.nn.Parameter(p.detach().to("cpu", copy=True), requires_grad=p.requires_grad)
    base = copy.deepcopy(model, memo)
    return base


class StopOnSignal:
    """utils.py:291-315 (SIGUSR1Callback): SIGUSR1 (a SLURM stop) or SIGINT sets
    a flag, and the training loop stops at the end of the current step
    (ZOTrainer.train). Installs the handlers on construction (main thread);
    close() puts the previous ones back."""

    def __init__(self, signals=(signal.SIGUSR1, signal.SIGINT)):
        self.signal_received = False
        self._prev = {s: signal.signal(s, self.handle_signal) for s in signals}

    def handle_signal(self, signum, frame) -> None:
        self.signal_received = True

    def close(self) -> None:
        for s, h in self._prev.items():
            signal.signal(s, h)
        self._prev = {}


class ZOTrainer(ZOTrainerMixin):
    """Minimal host of the ZO step: the reference's per-step contract
    (trainer.py:1206-1326) without the HF Trainer (no evaluation, saving or
    callbacks): zo_step, the NaN/inf loss filter, zo_update, global_step += 1,
    a loss record every step and a log line every 50 steps."""

    def __init__(self, model, args: ZOArguments, train_dataloader=None, *, base_model=None):
        self.args = args
        self.state = SimpleNamespace(global_step=0, epoch=0.0, log_history=[])
        self.zo_setup(model, train_dataloader, base_model=base_model)
        self.tr_loss = torch.zeros((), device=self.named_parameters_to_optim[0][1].device)
        self._last_logged = 0
        self._log_path = getattr(args, "zo_log_path", None)
        self._log_buf: List[tuple] = []
        self._graph = None
        if getattr(args, "zo_graph", False):
            from .graph import GraphedZOStep

            self._graph = GraphedZOStep(self)

    def _account(self, tr_loss_step) -> None:
        """The loss bookkeeping of trainer.py:1242-1250 (NaN/inf filter) on the device."""
        if self.args.logging_nan_inf_filter:
            bad = ~torch.isfinite(tr_loss_step)
            dec = self.tr_loss / (1 + self.state.global_step - self._last_logged)
            self.tr_loss = torch.where(bad, self.tr_loss + dec, self.tr_loss + tr_loss_step)
        else:
            self.tr_loss = self.tr_loss + tr_loss_step

    def _finish_step(self, tr_loss_step) -> None:
        self.state.global_step += 1
        if self.state.global_step % DIZO_INTERVAL == 0:
            self.state.log_history.append({"loss": round(tr_loss_step.item(), 4),
                                           "lr": self._get_learning_rate(),
                                           "step": self.state.global_step})
        self.loss_list.append(tr_loss_step)

    def training_step(self, inputs) -> torch.Tensor:
        """One optimisation step (trainer.py:1224-1326 with gradient_accumulation_steps = 1)."""
        if self._graph is not None:
            return self._graph_step(inputs)
        model = self.model
        tr_loss_step = self.zo_step(model, inputs)
        self._account(tr_loss_step)
        lr = self._get_learning_rate()
        self.zo_update(self.args, model)
        self._log_step(tr_loss_step, self._last_loss2, self._grad_value(), lr)
        self._finish_step(tr_loss_step)
        return tr_loss_step

    def _graph_step(self, inputs) -> torch.Tensor:
        """The same step replayed as a captured graph: zo_step and the update of
        zo_update with the seed, gradient and learning rate kept on the device
        (projected_grad is not read back; it stays None)."""
        args = self.args
        self.zo_random_seed = np.random.randint(1000000000)
        lr = self._get_learning_rate()
        tr_loss_step = self._graph.step(inputs, self.zo_random_seed, lr).clone()
        self.projected_grad = None
        g_dev = self._graph.d_prev_g.clone() if (self.zo_journal is not None or self._log_path) else None
        if self.zo_journal is not None:
            self.zo_journal.zo(self.zo_random_seed, g_dev, lr)
        self._log_step(tr_loss_step, None, g_dev, lr)
        self._account(tr_loss_step)
        if (self.state.global_step + 1) % DIZO_INTERVAL == 0 and args.enhanced:
            self._dizo_event(self.model, self.zo_random_seed)
        self.lr_scheduler.step()
        self._finish_step(tr_loss_step)
        return tr_loss_step

    def _log_step(self, loss1, loss2, g, lr: float) -> None:
        """Buffers one step's record (device scalars stay on the device)."""
        if not self._log_path:
            return
        self._log_buf.append((self.state.global_step + 1, self.zo_random_seed, loss1, loss2, g, float(lr)))
        if len(self._log_buf) >= DIZO_INTERVAL:
            self.flush_log()

    def flush_log(self) -> None:
        """Appends the buffered step records to zo_log_path as JSON lines."""
        if not self._log_path or not self._log_buf:
            return

        def host(x):
            if x is None:
                return None
            return float(x.item()) if torch.is_tensor(x) else float(x)

        with open(self._log_path, "a") as f:
            for step, seed, l1, l2, g, lr in self._log_buf:
                f.write(json.dumps({"step": int(step), "seed": int(seed), "loss1": host(l1), "loss2": host(l2),
                                    "projected_grad": host(g), "lr": lr}) + "\n")
        self._log_buf = []

    def train(self, batches, max_steps: Optional[int] = None, stop: Optional["StopOnSignal"] = None,
              checkpoint_dir: Optional[str] = None):
        """max_steps training steps over `batches`. With `stop`, a received signal
        ends the run at the end of the current step (trainer.py:1357 with
        utils.py:307-310); the pending fused work is applied and, given
        checkpoint_dir, a checkpoint is written (the reference asks for a save
        there). A re-iterable `batches` (a list, a DataLoader) is run again
        from its start when it ends, one epoch after another, as the
        reference's loop does (trainer.py:1186-1206); a one-shot iterator ends
        the run when it is exhausted. Returns the step losses."""
        n = max_steps if max_steps is not None else self.args.max_steps
        it = iter(batches)
        one_shot = it is batches
        for _ in range(n):
            try:
                inputs = next(it)
            except StopIteration:
                if one_shot:
                    break
                it = iter(batches)
                self.state.epoch += 1.0
                try:
                    inputs = next(it)
                except StopIteration:
                    raise DzError("train: batches is empty") from None
            self.training_step(inputs)
            if stop is not None and stop.signal_received:
                break
        self.zo_flush()
        self.flush_log()
        if stop is not None and stop.signal_received and checkpoint_dir:
            from .checkpoint import save_checkpoint

            save_checkpoint(self, checkpoint_dir)
        return [float(x) for x in self.loss_list]
