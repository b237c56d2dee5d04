"""Synthetic OPT-shaped models and prompt batches for tests and the benchmark.

No checkpoint or dataset is fetched. A model is ``transformers.OPTForCausalLM``
(the architecture the reference fine-tunes, run.py:174-181; shapes as in
ht_opt.py:103-125, 279-300) built on the meta device, materialised on the GPU
and initialised there by the library's own generator (stream DZ_STREAM_INIT),
the way HF initialises OPT: linear and embedding weights N(0, 0.02), biases
0, layer norms weight 1 / bias 0, the padding row of the token embedding 0.

Batches reproduce the layout the reference's collator produces for a binary
classification prompt (run.py:415-419 with train_as_classification,
utils.py:206-233): B examples x 2 candidates = 2B sequences, each the prompt
followed by one verbalizer token, left-padded with the pad id to a multiple
of 8, with attention_mask, labels (the correct candidate, repeated per
candidate), option_len = 1 and num_options = 2.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Iterator, List, Optional

import torch

from . import _lib as L
from .table import dtype_code

PAD_ID = 1
VERBALIZER_IDS = (6587, 372)  # two fixed candidate tokens (SST-2 style "terrible" / "great")


@dataclass(frozen=True)
class OPTShape:
    name: str
    layers: int
    d_model: int
    heads: int
    ffn: int
    vocab: int = 50272
    max_positions: int = 2048


SHAPES = {
    "opt-125m": OPTShape("opt-125m", 12, 768, 12, 3072),
    "opt-2.7b": OPTShape("opt-2.7b", 32, 2560, 32, 10240),
    "opt-13b": OPTShape("opt-13b", 40, 5120, 40, 20480),
    "opt-30b": OPTShape("opt-30b", 48, 7168, 56, 28672),
    # tiny shapes for tests
    "opt-tiny": OPTShape("opt-tiny", 2, 64, 4, 256, vocab=512, max_positions=128),
    "opt-mini": OPTShape("opt-mini", 4, 256, 4, 1024, vocab=4096, max_positions=256),
}


def opt_config(shape: OPTShape):
    from transformers import OPTConfig

    return OPTConfig(vocab_size=shape.vocab, hidden_size=shape.d_model, num_hidden_layers=shape.layers,
                     ffn_dim=shape.ffn, num_attention_heads=shape.heads,
                     max_position_embeddings=shape.max_positions, word_embed_proj_dim=shape.d_model,
                     pad_token_id=PAD_ID, dropout=0.0, attention_dropout=0.0, activation_dropout=0.0,
                     layerdrop=0.0, init_std=0.02)


def fill_normal_(t: torch.Tensor, seed: int, offset: int, std: float) -> torch.Tensor:
    """t <- std * z(seed, DZ_STREAM_INIT, offset + i), in place on the GPU."""
    if t.numel():
        with torch.cuda.device(t.device):
            L.call("dz_normals", int(seed), L.DZ_STREAM_INIT, int(offset), t.numel(), dtype_code(t.dtype),
                   t.data_ptr(), torch.cuda.current_stream(t.device).cuda_stream)
        t.mul_(std)
    return t


def build_opt(shape: str | OPTShape, dtype: torch.dtype = torch.float16, device="cuda", seed: int = 0,
              init_std: float = 0.02):
    """Random-init OPTForCausalLM of the given shape, in `dtype`, on `device`."""
    from transformers import OPTForCausalLM

    if isinstance(shape, str):
        shape = SHAPES[shape]
    cfg = opt_config(shape)
    with torch.device("meta"):
        model = OPTForCausalLM(cfg)
    model = model.to(dtype=dtype)
    model = model.to_empty(device=device)
    model.tie_weights()
    off = 0
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("layer_norm.weight"):
                p.fill_(1.0)
            elif name.endswith(".bias"):
                p.zero_()
            else:
                fill_normal_(p.data, seed, off, init_std)
                if name.endswith("embed_tokens.weight"):
                    p[PAD_ID].zero_()
            off += (p.numel() + 7) // 8 * 8
    model.eval()
    return model


def clone_model(model: torch.nn.Module) -> torch.nn.Module:
    """A full copy (theta0 resident on the device, as BASELINE configs C4/C5 keep it)."""
    import copy

    return copy.deepcopy(model)


def make_batch(batch: int, vocab: int, *, gen: torch.Generator, min_len: int = 32, max_len: int = 64,
               fixed_len: Optional[int] = None, device="cpu", pad_to_multiple_of: int = 8) -> Dict[str, torch.Tensor]:
    """One collated batch of `batch` examples x 2 candidates (2*batch rows).

    Prompt ids are uniform over the vocabulary; with fixed_len every row has
    fixed_len tokens (prompt fixed_len - 1 plus the verbalizer), else the
    prompt length is uniform in [min_len, max_len] and rows are left-padded.
    """
    rows, labels = [], []
    for _ in range(batch):
        if fixed_len is not None:
            n = fixed_len - 1
        else:
            n = int(torch.randint(min_len, max_len + 1, (1,), generator=gen))
        prompt = torch.randint(0, vocab, (n,), generator=gen)
        label = int(torch.randint(0, 2, (1,), generator=gen))
        for v in VERBALIZER_IDS:
            rows.append(torch.cat([prompt, torch.tensor([v % vocab])]))
            labels.append(label)
    L_ = max(len(r) for r in rows)
    if pad_to_multiple_of:
        L_ = (L_ + pad_to_multiple_of - 1) // pad_to_multiple_of * pad_to_multiple_of
    ids = torch.full((len(rows), L_), PAD_ID, dtype=torch.long)
    mask = torch.zeros((len(rows), L_), dtype=torch.long)
    for i, r in enumerate(rows):
        ids[i, L_ - len(r):] = r
        mask[i, L_ - len(r):] = 1
    out = {
        "input_ids": ids,
        "attention_mask": mask,
        "labels": torch.tensor(labels, dtype=torch.long),
        "option_len": torch.ones(len(rows), dtype=torch.long),
        "num_options": torch.full((len(rows),), 2, dtype=torch.long),
    }
    return {k: v.to(device) for k, v in out.items()}


def make_batches(n: int, batch: int, vocab: int, seed: int = 0, **kw) -> List[Dict[str, torch.Tensor]]:
    gen = torch.Generator().manual_seed(seed)
    return [make_batch(batch, vocab, gen=gen, **kw) for _ in range(n)]


class Cycle:
    """An endless loader over a fixed list of batches (restartable, like a DataLoader)."""

    def __init__(self, batches):
        self.batches = list(batches)

    def __iter__(self) -> Iterator:
        while True:
            yield from self.batches
