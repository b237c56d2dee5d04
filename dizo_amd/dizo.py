"""Drop-in DiZO layer-wise divergence projection on the HIP kernels.

``DiZO`` and ``dizo_trainer`` keep the reference's names, constructor
signatures, methods and state (luozoupi/DiZO, large_models/trainer.py):

  DiZO(model, norm_mode, exclude_list)                        trainer.py:378-403
    .apply_constraints(new, pre_trained, it, apply=False)     trainer.py:405-436
    .reverse_constraints(new, pre_trained)                    trainer.py:439-451
    ._project_ratio(new, anchor, it)                          trainer.py:453-465
    .perturb_gamma(delta, ts, zs, tau, zo_eps)                trainer.py:545-562
    .zo_forward(new, pre_trained, x, apply)                   trainer.py:564-614
    state: constraints (ParameterList, one gamma per projected tensor),
           alpha (dict), ts (list), init (bool)
  dizo_trainer(base_model, pgmloader, norm_mode, proj_lr, max_iters, exclude_list)
    .dizo_zo_iters(model, base_model, apply=False)            trainer.py:782-803
    .dizo_iters(model, base_model, apply=False)               trainer.py:805-830

The per-tensor loops of the reference become one launch over all projected
tensors: a group sum-of-squares pass for the norms, and APPLY / REVERSE
read-modify-write passes (REVERSE also returns the norms of the reversed
tensors, which the next ratio needs). The per-group scalar arithmetic on
gamma, the norms and alpha (clip, SPSA step, ratio) is evaluated elementwise
over a (G,) tensor with the reference's expressions, which gives each group
the reference's value.

The first-order path (``ENHANCED=fo``: ``DiZO.forward``, trainer.py:714-741,
and ``dizo_iters``, trainer.py:805-830) applies the projection in place with
an fp32 alpha (the reference's gamma is an fp32 Parameter there, so the
projected value is rounded to the model dtype once) inside an autograd
Function, runs the model forward with the graph, and in backward reduces
sum(fp32(dL/dtheta') * fp32(Delta)) per group with one kernel launch; the
tensors are then restored from a snapshot, because the reference evaluates
every iteration on a deep copy and never changes the model during the
search. Adam on gamma is torch's, as in the reference.

Differences from the reference, by design:
  * gamma noise (torch.normal in perturb_gamma, trainer.py:554) comes from
    the library's generator: stream DZ_STREAM_GAMMA keyed by the seed of the
    ZO step that triggered the event, one draw of G normals per SPSA
    iteration (``gamma_seed`` / draw counter);
  * norms accumulate in fp64 and round once (torch.norm accumulates in fp32):
    within one unit in the last place of the model dtype; likewise the
    first-order gradient's per-group sums (fp64 instead of fp32);
  * the first-order path works on the model itself (projected tensors
    snapshotted and restored) instead of a deep copy of the whole model.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence

import torch
from torch import nn

from . import _lib as L
from ._lib import DzError
from .table import ProjTable, normals
from .trainer import forward_wrap_with_option_len, option_len_loss

TAU, GAMMA_EPS, STEP_SIZE = 0.2, 0.1, 2  # trainer.py:590-592


class _ApplyFO(torch.autograd.Function):
    """theta' = R_T(fp32(R_T(theta - theta0)) * alpha + theta0), alpha = gamma / (norm + 1e-8),
    written in place into the projected tensors and recorded for autograd, as
    the reference's copy_ into the copied model records it (trainer.py:428-436
    under DiZO.forward, trainer.py:714-741)."""

    @staticmethod
    def forward(ctx, dizo, tab, saved_tab, norms, *args):
        G = dizo.G
        gammas, params = args[:G], args[G:]
        gam = torch.cat([g.detach().reshape(1) for g in gammas])
        denom = norms + 1e-8  # in the model dtype, as the reference's norms + 1e-8
        alpha = (gam / denom).contiguous()
        dizo._apply_alpha(tab, alpha)
        ctx.mark_dirty(*params)
        ctx.saved_tab = saved_tab
        ctx.save_for_backward(denom)
        return tuple(params)

    @staticmethod
    def backward(ctx, *grads):
        (denom,) = ctx.saved_tensors
        tab = ctx.saved_tab
        gs = [torch.zeros_like(t) if g is None else g.to(t.dtype).contiguous() for g, t in zip(grads, tab.tensors)]
        dot = torch.empty(len(gs), dtype=torch.float32, device=denom.device)
        tab.group_dot(gs, dot_f32=dot)  # dL/dalpha per group
        grad_gamma = dot / denom.to(torch.float32)  # d(gamma / denom) / d gamma
        return (None, None, None, None) + tuple(grad_gamma[i:i + 1] for i in range(len(gs))) + (None,) * len(gs)


class DiZO(nn.Module):
    """One gamma per projected tensor and the projection passes (trainer.py:378-614)."""

    @staticmethod
    def forward_wrap_with_option_len(self, input_ids=None, labels=None, option_len=None, num_options=None,
                                     return_dict=None, **kwargs):
        """trainer.py:470-542: the loss with the forward's autograd graph (``self`` is the model)."""
        return option_len_loss(self, True, input_ids, labels, option_len, num_options, return_dict, **kwargs)

    def __init__(self, model, norm_mode, exclude_list=[]) -> None:  # noqa: B006 (reference signature)
        super().__init__()
        if "l2" not in norm_mode:
            # trainer.py:460: the per-row L1 ("MARS") branch is unreachable with the
            # reference's only configuration, 'l2norm' (trainer.py:1168)
            raise DzError(f"norm_mode {norm_mode!r}: only the l2 norm is implemented")
        self.norm_mode = norm_mode
        self.exclude_list = list(exclude_list)
        self.threshold = nn.Hardtanh(0, 1)
        self.constraints_name: List[str] = []
        self.id_name_map: Dict[int, str] = {}
        constraints = []
        device = None
        for name, para in model.named_parameters():
            if name not in self.exclude_list and para.requires_grad:
                self.constraints_name.append(name)
                constraints.append(nn.Parameter(torch.Tensor([0]), requires_grad=True))
                self.id_name_map[len(self.constraints_name) - 1] = name
                if device is None and para.device.type == "cuda":
                    device = para.device
        if not constraints:
            raise DzError("DiZO: no projected tensors (every parameter is excluded)")
        self.constraints = nn.ParameterList(constraints)
        self._device = device if device is not None else torch.device("cuda", torch.cuda.current_device())
        self._set_gamma(torch.zeros(len(constraints), dtype=torch.float32, device=self._device))
        self.init = True
        self.times = 0
        self.alpha: Dict[str, torch.Tensor] = {}
        self.n = {}
        self.include_list: List[str] = []
        self.ts: List[torch.Tensor] = []
        # build state
        self.gamma_seed = 0
        self._draws = 0
        self._tab: Optional[ProjTable] = None
        self._tab_key = None
        self._alpha_vec: Optional[torch.Tensor] = None
        self._norms: Optional[torch.Tensor] = None  # norms of the current theta - theta0, when known
        self._in_event = False  # the driver vouches that theta is unchanged since _norms
        self.kernel_timer = None
        # first-order path: snapshot of the projected tensors and its table
        self._fo_saved: Optional[List[torch.Tensor]] = None
        self._fo_tab: Optional[ProjTable] = None
        self._fo_params: Optional[List[torch.Tensor]] = None
        self._fo_dirty = False
        # optional record of every pass that changes theta (checkpoint.ZOJournal)
        self.journal = None

    # ---------------------------------------------------------- gamma ----
    @property
    def G(self) -> int:
        return len(self.constraints_name)

    def _set_gamma(self, vec: torch.Tensor) -> None:
        """gamma lives in one (G,) tensor; each constraint Parameter views one element."""
        vec = vec.reshape(-1).contiguous()
        self._gamma = vec
        for i, p in enumerate(self.constraints):
            p.data = vec[i:i + 1]

    def gamma(self) -> torch.Tensor:
        """The (G,) gamma vector (constraint Parameters are views of it)."""
        return self._gamma

    # ---------------------------------------------------------- tables ---
    def _table(self, new: nn.Module, pre_trained: nn.Module) -> ProjTable:
        params = dict(new.named_parameters())
        anchors = dict(pre_trained.named_parameters())
        try:
            th = [params[n].data for n in self.constraints_name]
            t0 = [anchors[n].data for n in self.constraints_name]
        except KeyError as e:
            raise DzError(f"DiZO: parameter {e} missing from the model or its anchor") from None
        key = (tuple(t.data_ptr() for t in th), tuple(t.data_ptr() for t in t0))
        if self._tab is None or self._tab_key != key:
            if self._tab is not None:
                self._tab.close()
            self._tab = ProjTable(th, t0)
            self._tab_key = key
            self._norms = None
        return self._tab

    def _timed(self, name: str, tab: ProjTable, passes: int, fn) -> None:
        timer = self.kernel_timer
        if timer is None:
            fn()
        else:
            with timer.span(name, passes * tab.bytes_per_tensor_pass, [tab]):
                fn()

    def _group_norms(self, tab: ProjTable) -> torch.Tensor:
        """torch.norm(theta - theta0) of every group (trainer.py:455-457, 583), in T."""
        norms = torch.empty(self.G, dtype=tab.dtype, device=tab.device)
        self._timed("proj_sumsq", tab, 2, lambda: tab.group_sumsq(norm_T=norms))
        return norms

    def _ratio(self, norms: torch.Tensor) -> torch.Tensor:
        """trainer.py:464  constraint / (norms + 1e-8), per group."""
        return self._gamma / (norms + 1e-8)

    def _apply_alpha(self, tab: ProjTable, alpha: torch.Tensor) -> None:
        """Alpha in the model dtype (gamma in T, the ZO path): R(R(Delta alpha) + theta0);
        fp32 alpha (fp32 gamma, the first-order path): one rounding at the end."""
        alpha = alpha.contiguous()
        if alpha.dtype == tab.dtype:
            mode = L.DZ_PROJ_APPLY
        elif alpha.dtype == torch.float32:
            mode = L.DZ_PROJ_APPLY_F32ALPHA
        else:
            raise DzError(f"DiZO: alpha is {alpha.dtype} but the projected tensors are {tab.dtype}")
        self._timed("proj_apply", tab, 3, lambda: tab.project(alpha, mode))
        if self.journal is not None:
            self.journal.proj("apply" if mode == L.DZ_PROJ_APPLY else "apply_f32", alpha)
        self._alpha_vec = alpha
        self._norms = None
        self.alpha = {name: alpha[i:i + 1] for i, name in enumerate(self.constraints_name)}
        self.include_list = list(self.constraints_name)

    def _reverse(self, tab: ProjTable) -> torch.Tensor:
        """trainer.py:447-451 for every group, returning the norms of the reversed theta."""
        if self._alpha_vec is None:
            raise DzError("DiZO: reverse_constraints before apply_constraints")
        if self._alpha_vec.dtype != tab.dtype:
            raise DzError("DiZO: reverse_constraints after an fp32-alpha (first-order) apply is not supported")
        norms = torch.empty(self.G, dtype=tab.dtype, device=tab.device)
        self._timed("proj_reverse_sumsq", tab, 3,
                    lambda: tab.project(self._alpha_vec, L.DZ_PROJ_REVERSE_SUMSQ, norm_T=norms))
        if self.journal is not None:
            self.journal.proj("reverse", self._alpha_vec)
        self._norms = norms
        return norms

    @staticmethod
    def _freeze(model: nn.Module) -> None:
        for p in model.parameters():  # trainer.py:417, 444
            p.requires_grad = False

    # --------------------------------------------------- reference API ---
    def apply_constraints(self, new, pre_trained, constraint_iterator, apply=False):
        """trainer.py:405-436: theta <- theta0 + gamma / (||theta - theta0|| + 1e-8) * (theta - theta0)."""
        tab = self._table(new, pre_trained)
        gam = [next(constraint_iterator) for _ in range(self.G)]
        if any(g.data.data_ptr() != self._gamma[i:i + 1].data_ptr() for i, g in enumerate(gam)):
            self._set_gamma(torch.cat([g.data.reshape(1) for g in gam]))
        trusted = self._in_event and self._norms is not None
        norms = self._norms if trusted else self._group_norms(tab)
        self._freeze(new)
        self._apply_alpha(tab, self._ratio(norms))

    def reverse_constraints(self, new, pre_trained):
        """trainer.py:439-451: theta <- theta0 + (theta - theta0) / alpha."""
        tab = self._table(new, pre_trained)
        self._freeze(new)
        self._reverse(tab)

    # ------------------------------------------- supplied / searched -----
    def apply_ratio(self, new, pre_trained, alpha) -> None:
        """theta <- theta0 + alpha (theta - theta0) for every projected tensor with a
        supplied ratio (one number for all groups, or one per group; the "alpha
        supplied" form, e.g. a fixed 0.9 per layer). alpha is rounded to the model
        dtype and applied as trainer.py:428-436 applies gamma / (norm + 1e-8)."""
        tab = self._table(new, pre_trained)
        a = torch.as_tensor(alpha, dtype=torch.float64).reshape(-1)
        if a.numel() == 1:
            a = a.expand(self.G)
        if a.numel() != self.G:
            raise DzError(f"DiZO.apply_ratio: {a.numel()} ratios for {self.G} groups")
        self._freeze(new)
        self._apply_alpha(tab, a.float().to(tab.dtype).to(tab.device).contiguous())

    def apply_gamma(self, new, pre_trained, gamma) -> None:
        """apply_constraints with supplied gamma (target norms ||theta - theta0||;
        one number for all groups, or one per group; the "gamma supplied" form).
        A Python number or list is an fp32 gamma, as the reference's constraint
        Parameters are (alpha is then fp32 and the result is rounded once); a
        tensor keeps its dtype."""
        if torch.is_tensor(gamma):
            g = gamma.detach().reshape(-1).to(self._device)
        else:
            g = torch.as_tensor(gamma, dtype=torch.float32, device=self._device).reshape(-1)
        if g.numel() == 1:
            g = g.expand(self.G)
        if g.numel() != self.G:
            raise DzError(f"DiZO.apply_gamma: {g.numel()} values for {self.G} groups")
        self._set_gamma(g.clone())
        self.apply_constraints(new, pre_trained, iter(self.constraints))

    def grid_search(self, new, pre_trained, x, candidates: Sequence[float]):
        """Searched ratio: the loss on batch x at each candidate ratio (the same for
        every group, e.g. 8 values in [0.5, 1.0]), each evaluated from the same
        theta (the projected tensors are restored exactly between candidates),
        then the candidate with the lowest loss (the first of equals) applied.
        Returns (chosen ratio, losses)."""
        if len(candidates) == 0:
            raise DzError("DiZO.grid_search: no candidates")
        self.fo_restore()
        self._fo_snapshot(new, pre_trained)
        losses = []
        with torch.no_grad():
            for r in candidates:
                if self.journal is not None:
                    self.journal.mark()  # the candidate's apply is undone below
                self.apply_ratio(new, pre_trained, r)
                self._fo_dirty = True
                losses.append(self._loss(new, x).reshape(()).float())
                self.fo_restore()
            best = int(torch.stack(losses).argmin().item())
            self.apply_ratio(new, pre_trained, candidates[best])
        self.last_losses = tuple(losses)
        return float(candidates[best]), losses

    def _project_ratio(self, new, anchor, constraint_iterator):
        """trainer.py:453-465 for one projected tensor `new` with anchor `anchor`."""
        if self._tab is None:
            raise DzError("DiZO._project_ratio: no projection table yet (call apply_constraints first)")
        ptrs = [t.data_ptr() for t in self._tab.tensors]
        try:
            i = ptrs.index(new.data_ptr())
        except ValueError:
            raise DzError("DiZO._project_ratio: tensor is not one of the projected tensors") from None
        constraint = next(constraint_iterator)
        norms = self._group_norms(self._tab)
        return constraint / (norms[i] + 1e-8)

    def _draw_gamma_z(self, dtype: torch.dtype) -> torch.Tensor:
        """G standard normals for one perturb_gamma draw (trainer.py:554)."""
        z = normals(self.gamma_seed, L.DZ_STREAM_GAMMA, self._draws * self.G, self.G, dtype, self._device)
        self._draws += 1
        return z

    def perturb_gamma(self, delta, ts=None, zs=None, tau=None, zo_eps=None):
        """trainer.py:545-562 over all groups: gamma <- gamma + delta * z * zo_eps,
        z ~ N(0, 1) clipped to +-(tau / zo_eps) * ts (drawn when zs is None)."""
        if zs is None:
            ts_v = torch.stack([t.reshape(()) for t in ts]) if isinstance(ts, (list, tuple)) else ts
            z = self._draw_gamma_z(self._gamma.dtype)
            zs = torch.clip(z, (-tau / zo_eps) * ts_v, (tau / zo_eps) * ts_v)
        self._set_gamma(self._gamma + delta * zs * zo_eps)
        return zs

    def _loss(self, model, x):
        return forward_wrap_with_option_len(model, **x, return_dict=True).loss

    def zo_forward(self, new=None, pre_trained=None, x=None, apply=False):
        """trainer.py:564-614: one SPSA iteration on gamma (apply=False), or the final
        apply_constraints with the current gamma (apply=True)."""
        if apply:
            self.apply_constraints(new, pre_trained, iter(self.constraints), apply=True)
            return
        with torch.no_grad():
            tab = self._table(new, pre_trained)
            trusted = self._in_event and self._norms is not None
            ts_v = self._norms if trusted else self._group_norms(tab)
            ts_v = ts_v.clone()
            if self.init:
                self._set_gamma(ts_v.clone())
            zs = self.perturb_gamma(1, ts=ts_v, tau=TAU, zo_eps=GAMMA_EPS)
            self._freeze(new)
            self._apply_alpha(tab, self._ratio(ts_v))
            loss1 = self._loss(new, x)
            n1 = self._reverse(tab)
            self.perturb_gamma(-2, ts=ts_v, zs=zs, tau=TAU, zo_eps=GAMMA_EPS)
            self._apply_alpha(tab, self._ratio(n1))
            loss2 = self._loss(new, x)
            self._reverse(tab)
            self.perturb_gamma(1, ts=ts_v, zs=zs, tau=TAU, zo_eps=GAMMA_EPS)
            grad = (loss1 - loss2) / (2 * GAMMA_EPS)
            new_gamma = torch.clip(self._gamma - STEP_SIZE * ts_v * grad * zs, (1 - TAU) * ts_v, (1 + TAU) * ts_v)
            self._set_gamma(new_gamma)
        self.ts = [ts_v[i] for i in range(self.G)]
        self.last_losses = (loss1, loss2)

    # ------------------------------------------------ first-order path --
    def _fo_snapshot(self, new, pre_trained):
        """Copies the projected tensors into the snapshot (allocated once)."""
        params = dict(new.named_parameters())
        anchors = dict(pre_trained.named_parameters())
        ps = [params[n] for n in self.constraints_name]
        if self._fo_saved is None or any(a.shape != b.shape for a, b in zip(self._fo_saved, ps)):
            if self._fo_tab is not None:
                self._fo_tab.close()
            self._fo_saved = [torch.empty_like(p.data) for p in ps]
            self._fo_tab = ProjTable(self._fo_saved, [anchors[n].data for n in self.constraints_name])
        with torch.no_grad():
            for b, p in zip(self._fo_saved, ps):
                b.copy_(p.data)
        self._fo_params = ps
        if self.journal is not None:
            self.journal.mark()
        return ps

    def fo_restore(self) -> None:
        """Puts the projected tensors back to the snapshot after a first-order
        iteration and drops their autograd history."""
        if self._fo_dirty:
            with torch.no_grad():
                for p, b in zip(self._fo_params, self._fo_saved):
                    p.detach_()
                    p.requires_grad_(False)
                    p.data.copy_(b)
            self._fo_dirty = False
            self._norms = None
            if self.journal is not None:
                self.journal.rollback()

    def forward(self, new=None, pre_trained=None, x=None, apply=False):
        """trainer.py:714-741: with apply, the final projection; otherwise the
        first-order objective loss + 1e-3 * sum |gamma| on the projected model,
        differentiable with respect to gamma."""
        self.fo_restore()
        if apply:
            self.apply_constraints(new, pre_trained, iter(self.constraints), apply=True)
            return None
        tab = self._table(new, pre_trained)
        params = self._fo_snapshot(new, pre_trained)
        norms = self._group_norms(tab)
        self._freeze(new)
        _ApplyFO.apply(self, tab, self._fo_tab, norms, *list(self.constraints), *params)
        self._fo_dirty = True
        self._norms = None
        out = self.forward_wrap_with_option_len(new, **x, return_dict=True)
        return out.loss + 1e-3 * sum(p.abs().sum() for p in self.constraints.parameters())

    def close(self) -> None:
        self.fo_restore()
        for name in ("_tab", "_fo_tab"):
            tab = getattr(self, name)
            if tab is not None:
                tab.close()
                setattr(self, name, None)


class dizo_trainer:  # noqa: N801 (reference name)
    """Driver of the DiZO event (trainer.py:744-830)."""

    def __init__(self, base_model, pgmloader, norm_mode, proj_lr, max_iters, exclude_list=[]) -> None:  # noqa: B006
        self.proj_lr = proj_lr
        self.max_iters = max_iters
        self.exclude_list = exclude_list
        self.dizo = DiZO(base_model, norm_mode=norm_mode, exclude_list=exclude_list)
        self.device = self.dizo._device
        self.pre_trained = base_model
        self.pgm_optimizer = torch.optim.Adam(self.dizo.parameters(), lr=self.proj_lr)
        self.pgmloader = pgmloader
        self.dataset_iterator = iter(self.pgmloader) if pgmloader is not None else None
        self.criterion = torch.nn.CrossEntropyLoss()
        self.i = 0
        self.gamma_seed = 0
        self.batches_drawn = 0  # gamma-search batches taken so far (for checkpoints)

    def bind_model(self, model) -> None:
        """Registers the projection table of (model, anchor) ahead of the first event."""
        self.dizo._table(model, self.pre_trained)

    def _draw(self):
        try:
            data = next(self.dataset_iterator)
        except StopIteration:
            self.dataset_iterator = iter(self.pgmloader)
            data = next(self.dataset_iterator)
        self.batches_drawn += 1
        return data

    def _next_batch(self):
        if self.pgmloader is None:
            raise DzError("dizo_trainer: no data loader for the gamma search")
        data = self._draw()
        return {k: (v.to(self.device) if torch.is_tensor(v) else v) for k, v in data.items()}

    def rewind_loader(self, drawn: int) -> None:
        """Restarts the gamma search's loader and skips the `drawn` batches a
        checkpointed run had taken (exact for a loader with a fixed order)."""
        self.batches_drawn = 0
        if self.pgmloader is None:
            return
        self.dataset_iterator = iter(self.pgmloader)
        for _ in range(drawn):
            self._draw()

    def dizo_zo_iters(self, model, base_model, apply=False):
        """trainer.py:782-803: max_iters SPSA iterations on gamma, then the final apply."""
        dz = self.dizo
        dz.gamma_seed = self.gamma_seed
        dz._draws = 0
        dz._norms = None
        dz._in_event = True  # between the passes below nothing else writes theta
        try:
            if not apply:
                self.count = 0
                dz.init = True
                while self.count < self.max_iters:
                    data = self._next_batch()
                    dz.zo_forward(model, base_model, x=data)
                    dz.init = False
                    self.count += 1
            dz.zo_forward(model, self.pre_trained, apply=True)
        finally:
            dz._in_event = False
            dz._norms = None
        self.i += 1

    def dizo_grid_iters(self, model, base_model, candidates: Sequence[float]) -> float:
        """The searched-ratio event: one batch from the loader, the loss at each
        candidate ratio, the best one applied (DiZO.grid_search). Returns the ratio."""
        data = self._next_batch()
        r, _ = self.dizo.grid_search(model, base_model, data, candidates)
        self.i += 1
        return r

    def dizo_iters(self, model, base_model, apply=False):
        """trainer.py:805-830: max_iters first-order iterations (Adam on gamma,
        lr proj_lr), then the final apply."""
        dz = self.dizo
        if not apply:
            self.count = 0
            with torch.enable_grad():
                while self.count < self.max_iters:
                    data = self._next_batch()
                    pgm_loss = dz(model, base_model, x=data)
                    self.pgm_optimizer.zero_grad()
                    pgm_loss.backward()
                    self.pgm_optimizer.step()
                    dz.fo_restore()
                    self.count += 1
        dz(model, self.pre_trained, apply=True)
        self.i += 1

    def close(self) -> None:
        self.dizo.close()
