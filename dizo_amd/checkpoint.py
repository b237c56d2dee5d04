"""ZO checkpoint and replay (replaces the HF checkpointing of run.py:466-479 and
trainer.py:1072-1095 for the zeroth-order path).

A ZO run changes the trainable tensors only through:

  * ZO steps (trainer.py:1570-1617): +eps z, -2 eps z, +eps z, then
    -lr (g z), with z regenerated from the step's seed;
  * DiZO projection passes (trainer.py:405-451): apply with alpha per
    group (in the model dtype, or fp32 on the first-order path), and
    reverse with the alpha of the last apply.

``ZOJournal`` records them in order: ``["zo", seed, g, lr]`` per step and
``[mode, alpha]`` per projection pass. The projections inside a first-order
iteration are dropped, because the iteration ends by restoring the snapshot
taken before it. Replaying a journal on the weights the run started from
recomputes the run's weights bit for bit, without a forward: the same kernels
apply the same per-element operations in the same order. Fused passes apply
the same per-element operations as separate ones, so a replay can use the
fused forms: 2 passes per ZO step and 1 per projection op. At OPT-13B a
thousand steps replay in about 20 s, from about 40 bytes of journal per step.

A checkpoint directory holds:

  theta.safetensors   every parameter of the model by name, and the anchors
                      (theta0) of the projected tensors as "anchor:<name>"
  state.json          step counter, numpy RNG state (the step seeds come from
                      np.random, trainer.py:1577), LR scheduler, DiZO state
                      (gamma, the alpha of the last apply, the first-order
                      Adam state, batches drawn by the gamma search) and the
                      loss bookkeeping
  journal.json        the journal of the whole run, when one was kept

Resuming from a checkpoint continues the run exactly. It needs the same
model, batches and arguments, and a deterministic data order: the gamma
search's loader is advanced by the number of batches it had drawn.
"""
from __future__ import annotations

import json
import os
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib as L
from ._lib import DzError

FORMAT = "dizo-amd-zo-journal"
# 3: z drawn from Philox4x32-7 with the counter words (stream, q lo, 0, q hi).
# Journals and checkpoints of earlier versions (version 1: Philox4x32-10;
# version 2: counter (q lo, q hi, stream, 0)) do not replay on this library.
VERSION = 3
STATE_FORMAT = "dizo-amd-zo-checkpoint"
PROJ_MODES = {"apply": L.DZ_PROJ_APPLY, "apply_f32": L.DZ_PROJ_APPLY_F32ALPHA, "reverse": L.DZ_PROJ_REVERSE}
_DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}


def _dtype_name(dt: torch.dtype) -> str:
    for k, v in _DTYPES.items():
        if v == dt:
            return k
    raise DzError(f"unsupported dtype {dt}")


class ZOJournal:
    """Ordered record of the operations that changed the trainable tensors."""

    def __init__(self, layout: Sequence[Tuple[str, int, str]], eps: float, projected: Sequence[str] = ()):
        self.layout = [(str(n), int(k), str(d)) for n, k, d in layout]  # (name, numel, dtype) in z order
        self.eps = float(eps)
        self.projected = list(projected)
        self.ops: List[list] = []
        self._mark: Optional[int] = None

    @classmethod
    def for_params(cls, named: Sequence[Tuple[str, torch.Tensor]], eps: float, projected: Sequence[str] = ()):
        return cls([(n, p.numel(), _dtype_name(p.dtype)) for n, p in named], eps, projected)

    # ------------------------------------------------------- recording ----
    def zo(self, seed: int, g, lr: float) -> None:
        """One ZO step. g is the projected gradient as a float, or as a 0-dim device
        tensor (a captured step keeps it on the device; it is read when saved)."""
        self.ops.append(["zo", int(seed), g, float(lr)])

    def proj(self, mode: str, alpha: torch.Tensor) -> None:
        if mode not in PROJ_MODES:
            raise DzError(f"journal: unknown projection mode {mode!r}")
        self.ops.append([mode, alpha.detach().clone()])

    def mark(self) -> None:
        """Start of a first-order iteration (its projections are undone by a snapshot restore)."""
        self._mark = len(self.ops)

    def rollback(self) -> None:
        """The snapshot taken at mark() was restored: drop what was recorded since."""
        if self._mark is not None:
            del self.ops[self._mark:]
            self._mark = None

    @property
    def steps(self) -> int:
        return sum(1 for op in self.ops if op[0] == "zo")

    # ------------------------------------------------------------- I/O ----
    def to_json(self) -> Dict[str, Any]:
        ops = []
        for op in self.ops:
            if op[0] == "zo":
                g = op[2]
                ops.append(["zo", op[1], float(g.item() if torch.is_tensor(g) else g), op[3]])
            else:
                a = op[1]
                ops.append([op[0], _dtype_name(a.dtype), [float(x) for x in a.float().cpu().tolist()]])
        return {"format": FORMAT, "version": VERSION, "eps": self.eps, "layout": self.layout,
                "projected": self.projected, "ops": ops}

    @classmethod
    def from_json(cls, d: Dict[str, Any]) -> "ZOJournal":
        if d.get("format") != FORMAT or d.get("version") != VERSION:
            raise DzError(f"not a {FORMAT} v{VERSION} journal: {d.get('format')!r} v{d.get('version')!r}")
        j = cls([tuple(x) for x in d["layout"]], d["eps"], d.get("projected", []))
        for op in d["ops"]:
            if op[0] == "zo":
                j.ops.append(["zo", int(op[1]), float(op[2]), float(op[3])])
            elif op[0] in PROJ_MODES:
                j.ops.append([op[0], torch.tensor(op[2], dtype=torch.float32).to(_DTYPES[op[1]])])
            else:
                raise DzError(f"journal: unknown op {op[0]!r}")
        return j

    def save(self, path: str) -> None:
        tmp = path + ".tmp"
        with open(tmp, "w") as f:
            json.dump(self.to_json(), f)
        os.replace(tmp, path)

    @classmethod
    def load(cls, path: str) -> "ZOJournal":
        with open(path) as f:
            return cls.from_json(json.load(f))


def replay_plan(ops: Sequence[list]) -> List[tuple]:
    """The passes that reproduce a journal, fused as the trainer fuses them:
    ("perturb", seed, scale), ("restore_update_perturb", (seed, g, lr), next_seed),
    ("restore_update", (seed, g, lr)) and ("proj", mode, alpha)."""
    plan: List[tuple] = []
    pending = None
    for op in ops:
        if op[0] == "zo":
            _, seed, g, lr = op
            if pending is None:
                plan.append(("perturb", seed, 1.0))
            else:
                plan.append(("restore_update_perturb", pending, seed))
            plan.append(("perturb", seed, -2.0))
            pending = (seed, g, lr)
        else:
            if pending is not None:
                plan.append(("restore_update", pending))
                pending = None
            plan.append(("proj", op[0], op[1]))
    if pending is not None:
        plan.append(("restore_update", pending))
    return plan


def _check_layout(journal: ZOJournal, named: Sequence[Tuple[str, torch.Tensor]]) -> None:
    got = [(n, p.numel(), _dtype_name(p.dtype)) for n, p in named]
    if got != journal.layout:
        for i, (a, b) in enumerate(zip(got, journal.layout)):
            if a != b:
                raise DzError(f"journal layout differs at tensor {i}: model {a} vs journal {b}")
        raise DzError(f"journal layout has {len(journal.layout)} tensors, the model {len(got)}")


def replay(model: torch.nn.Module, journal: ZOJournal, base_model: Optional[torch.nn.Module] = None,
           upto: Optional[int] = None) -> int:
    """Applies the journal's operations (the first `upto` ZO steps and the
    projections recorded before the next one) to the model's trainable
    tensors in place. base_model supplies theta0 for projection ops. Returns
    the number of ZO steps replayed."""
    from .table import ProjTable
    from .trainer import _ZOTables

    # by the journal's names: a DiZO event clears requires_grad on every
    # parameter (trainer.py:417), so the trainable set cannot be re-derived
    params = dict(model.named_parameters())
    try:
        named = [(n, params[n]) for n, _, _ in journal.layout]
    except KeyError as e:
        raise DzError(f"journal tensor {e} is not a parameter of the model") from None
    _check_layout(journal, named)
    ops = journal.ops
    if upto is not None:
        n, cut = 0, len(ops)
        for i, op in enumerate(ops):
            if op[0] == "zo":
                if n == upto:
                    cut = i
                    break
                n += 1
        ops = ops[:cut]
    eps = journal.eps
    tabs = _ZOTables(named)
    ptab = None
    try:
        for step in replay_plan(ops):
            kind = step[0]
            if kind == "perturb":
                for t, _ in tabs.tables:
                    t.perturb(step[1], step[2], eps)
            elif kind == "restore_update_perturb":
                (seed, g, lr), nxt = step[1], step[2]
                for t, _ in tabs.tables:
                    t.restore_update_perturb(seed, nxt, eps, g, lr)
            elif kind == "restore_update":
                seed, g, lr = step[1]
                for t, _ in tabs.tables:
                    t.restore_update(seed, eps, g, lr)
            else:
                if ptab is None:
                    if base_model is None:
                        raise DzError("replay: the journal has projection ops; pass base_model (theta0)")
                    params = dict(model.named_parameters())
                    anchors = dict(base_model.named_parameters())
                    ptab = ProjTable([params[n].data for n in journal.projected],
                                     [anchors[n].data for n in journal.projected])
                alpha = step[2].to(ptab.device)
                ptab.project(alpha.contiguous(), PROJ_MODES[step[1]])
    finally:
        tabs.close()
        if ptab is not None:
            ptab.close()
    return sum(1 for op in ops if op[0] == "zo")


# ------------------------------------------------------------ checkpoints ----
def _np_state() -> list:
    name, keys, pos, has_gauss, cached = np.random.get_state()
    return [name, [int(k) for k in keys], int(pos), int(has_gauss), float(cached)]


def _set_np_state(s: list) -> None:
    np.random.set_state((s[0], np.array(s[1], dtype=np.uint32), int(s[2]), int(s[3]), float(s[4])))


def _vec(t: Optional[torch.Tensor]):
    if t is None:
        return None
    return {"dtype": _dtype_name(t.dtype), "values": [float(x) for x in t.detach().float().cpu().tolist()]}


def _unvec(d, device) -> Optional[torch.Tensor]:
    if d is None:
        return None
    return torch.tensor(d["values"], dtype=torch.float32).to(_DTYPES[d["dtype"]]).to(device)


def _adam_state(opt: torch.optim.Optimizer) -> Dict[str, Any]:
    sd = opt.state_dict()
    state = {}
    for k, st in sd["state"].items():
        state[str(k)] = {n: (_vec(v.reshape(-1)) if torch.is_tensor(v) else v) for n, v in st.items()}
    return {"state": state, "param_groups": sd["param_groups"]}


def _load_adam_state(opt: torch.optim.Optimizer, d: Dict[str, Any], device) -> None:
    state = {}
    params = [p for g in opt.param_groups for p in g["params"]]
    for k, st in d["state"].items():
        p = params[int(k)]
        entry = {}
        for n, v in st.items():
            if isinstance(v, dict):
                t = _unvec(v, device)
                entry[n] = t.reshape(p.shape) if t.numel() == p.numel() else t.reshape(())
            else:
                entry[n] = v
        if "step" in entry and not torch.is_tensor(entry["step"]):
            entry["step"] = torch.tensor(float(entry["step"]))
        elif "step" in entry:
            entry["step"] = entry["step"].cpu().float().reshape(())
        state[int(k)] = entry
    opt.load_state_dict({"state": state, "param_groups": d["param_groups"]})


def save_checkpoint(trainer, path: str) -> None:
    """Writes theta, the run state and the journal of a ZOTrainerMixin host
    (call between steps; pending fused work is applied first). Each file is
    replaced atomically, but the files are replaced one after another: save
    into a fresh directory (one per step, say) so that an interrupted save
    cannot leave files of two saves side by side."""
    from safetensors.torch import save_file

    trainer.zo_flush()
    os.makedirs(path, exist_ok=True)
    # copies, never views: parameters may share one storage (the fused k/v/q
    # buffer of dizo_amd.fused_layers), which safetensors refuses, and .cpu()
    # of a CPU tensor would return the tensor itself
    tensors = {n: p.detach().to("cpu", copy=True).contiguous() for n, p in trainer.model.named_parameters()}
    dtr = getattr(trainer, "dizo_trainer", None) if trainer.args.enhanced else None
    if dtr is not None:
        anchors = dict(trainer.base_model.named_parameters())
        for n in dtr.dizo.constraints_name:
            tensors["anchor:" + n] = anchors[n].detach().to("cpu", copy=True).contiguous()
    # each file is written to a temporary name and renamed into place, so an
    # interrupted save never leaves a partial file beside an older state
    tmp = os.path.join(path, "theta.safetensors.tmp")
    save_file(tensors, tmp)
    os.replace(tmp, os.path.join(path, "theta.safetensors"))
    sched = trainer.lr_scheduler
    state: Dict[str, Any] = {
        "format": STATE_FORMAT, "version": VERSION,
        "global_step": int(trainer.state.global_step),
        "numpy_rng": _np_state(),
        "scheduler": {"last_epoch": int(sched.last_epoch), "last_lr": [float(x) for x in sched.get_last_lr()],
                      "base_lrs": [float(x) for x in sched.base_lrs]},
        "optimizer_lr": [float(g["lr"]) for g in trainer.optimizer.param_groups],
        "zo_random_seed": trainer.zo_random_seed,
        "tr_loss": float(trainer.tr_loss) if torch.is_tensor(getattr(trainer, "tr_loss", None)) else None,
        "last_logged": int(getattr(trainer, "_last_logged", 0)),
        "loss_list": [float(x) for x in getattr(trainer, "loss_list", [])],
        "enhanced": trainer.args.enhanced,
    }
    if dtr is not None:
        dz = dtr.dizo
        state["dizo"] = {
            "gamma": _vec(dz.gamma()), "alpha": _vec(dz._alpha_vec), "init": bool(dz.init),
            "ts": _vec(torch.stack([t.reshape(()) for t in dz.ts])) if dz.ts else None,
            "events": int(dtr.i), "gamma_seed": int(dtr.gamma_seed),
            "batches_drawn": int(getattr(dtr, "batches_drawn", 0)),
            "adam": _adam_state(dtr.pgm_optimizer),
        }
    tmp = os.path.join(path, "state.json.tmp")
    with open(tmp, "w") as f:
        json.dump(state, f)
    os.replace(tmp, os.path.join(path, "state.json"))
    journal = getattr(trainer, "zo_journal", None)
    if journal is not None:
        journal.save(os.path.join(path, "journal.json"))


def load_checkpoint(trainer, path: str) -> None:
    """Restores a checkpoint into a ZOTrainerMixin host set up on a model of the
    same architecture and the same arguments (zo_setup done): every parameter
    (copied in place, so the kernels' tables stay valid), the anchors of the
    projected tensors, the numpy RNG, the step counter, the LR scheduler, the
    DiZO state and the journal."""
    from safetensors.torch import load_file

    with open(os.path.join(path, "state.json")) as f:
        state = json.load(f)
    if state.get("format") != STATE_FORMAT or state.get("version") != VERSION:
        raise DzError(f"{path}: not a {STATE_FORMAT} v{VERSION} checkpoint")
    if state.get("enhanced") != trainer.args.enhanced:
        raise DzError(f"checkpoint was written with enhanced={state.get('enhanced')!r}, "
                      f"the trainer has {trainer.args.enhanced!r}")
    trainer.zo_flush()
    tensors = load_file(os.path.join(path, "theta.safetensors"))
    with torch.no_grad():
        for n, p in trainer.model.named_parameters():
            if n not in tensors:
                raise DzError(f"checkpoint has no tensor {n!r}")
            src = tensors[n]
            if src.shape != p.shape or src.dtype != p.dtype:
                raise DzError(f"checkpoint tensor {n!r} is {tuple(src.shape)} {src.dtype}, "
                              f"the model's {tuple(p.shape)} {p.dtype}")
            p.data.copy_(src)
    trainer.state.global_step = int(state["global_step"])
    _set_np_state(state["numpy_rng"])
    sched = trainer.lr_scheduler
    sched.last_epoch = int(state["scheduler"]["last_epoch"])
    sched._last_lr = list(state["scheduler"]["last_lr"])
    sched.base_lrs = list(state["scheduler"]["base_lrs"])
    for g, lr in zip(trainer.optimizer.param_groups, state["optimizer_lr"]):
        g["lr"] = lr
    trainer.zo_random_seed = state.get("zo_random_seed")
    if state.get("tr_loss") is not None and torch.is_tensor(getattr(trainer, "tr_loss", None)):
        trainer.tr_loss = torch.tensor(state["tr_loss"], dtype=trainer.tr_loss.dtype, device=trainer.tr_loss.device)
    trainer._last_logged = int(state.get("last_logged", 0))
    if hasattr(trainer, "loss_list"):
        trainer.loss_list = [torch.tensor(x) for x in state.get("loss_list", [])]
    dz_state = state.get("dizo")
    if dz_state is not None:
        dtr = trainer.dizo_trainer
        dz = dtr.dizo
        anchors = dict(trainer.base_model.named_parameters())
        with torch.no_grad():
            for n in dz.constraints_name:
                anchors[n].data.copy_(tensors["anchor:" + n])
        dev = dz._device
        dz.fo_restore()
        dz._set_gamma(_unvec(dz_state["gamma"], dev))
        dz._alpha_vec = _unvec(dz_state["alpha"], dev)
        if dz._alpha_vec is not None:
            dz.alpha = {name: dz._alpha_vec[i:i + 1] for i, name in enumerate(dz.constraints_name)}
            dz.include_list = list(dz.constraints_name)
        dz.init = bool(dz_state["init"])
        ts = _unvec(dz_state["ts"], dev)
        dz.ts = [] if ts is None else [ts[i] for i in range(ts.numel())]
        dz._norms = None
        dtr.i = int(dz_state["events"])
        dtr.gamma_seed = int(dz_state["gamma_seed"])
        _load_adam_state(dtr.pgm_optimizer, dz_state["adam"], dev)
        dtr.rewind_loader(int(dz_state["batches_drawn"]))
    jpath = os.path.join(path, "journal.json")
    if os.path.exists(jpath):
        trainer.zo_journal = ZOJournal.load(jpath)
        if getattr(trainer, "dizo_trainer", None) is not None and trainer.args.enhanced:
            trainer.dizo_trainer.dizo.journal = trainer.zo_journal
