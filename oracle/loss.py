"""float64 brute-force restatement of the ZO forward's loss (test oracle only).

trainer.py:1446-1522 (forward_wrap_with_option_len), classification branch:
for every row r (one candidate of one example), the option tokens are the
last option_len[r] positions (all positions when option_len[r] is 0: the
reference masks with ``shift_labels[i, :-len]``, and [:-0] is an empty
slice, trainer.py:1473-1475); each option token t at position j is predicted
by the logits at position j - 1; pad ids (config.pad_token_id) are never
targets. The row score is the mean over its option tokens of
log_softmax(logits[j - 1])[t]. Rows are grouped into examples of
num_options candidates; the loss is the mean over examples of the
cross-entropy of the example's scores against its label (labels repeat per
candidate; the first of each group is used). Equal num_options take the
batched CrossEntropyLoss path (mean over examples); unequal ones the loop
path (sum of per-example losses / count): the same value.
"""
from __future__ import annotations

import math
from typing import Sequence

import numpy as np


def row_scores(logits: np.ndarray, input_ids: np.ndarray, option_len: Sequence[int], pad_id: int) -> np.ndarray:
    """Mean option-token log-probability per row, in float64 (loops, no vectorisation)."""
    rows, L, V = logits.shape
    out = np.zeros(rows, dtype=np.float64)
    for r in range(rows):
        total, count = 0.0, 0
        ol = int(option_len[r])
        for j in range(L - ol if ol > 0 else 1, L):
            if j < 1:
                continue
            tok = int(input_ids[r, j])
            if tok == pad_id:
                continue
            x = logits[r, j - 1].astype(np.float64)
            m = x.max()
            lse = m + math.log(np.exp(x - m).sum())
            total += x[tok] - lse
            count += 1
        out[r] = total / count if count else float("nan")
    return out


def classification_loss(logits: np.ndarray, input_ids: np.ndarray, labels: Sequence[int],
                        option_len: Sequence[int], num_options: Sequence[int], pad_id: int) -> float:
    scores = row_scores(logits, input_ids, option_len, pad_id)
    losses, start = [], 0
    while start < len(num_options):
        k = int(num_options[start])
        s = scores[start:start + k]
        lab = int(labels[start])
        m = s.max()
        losses.append(-(s[lab] - (m + math.log(np.exp(s - m).sum()))))
        start += k
    return float(np.mean(losses))
