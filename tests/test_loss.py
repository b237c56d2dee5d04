"""The ZO forward's loss (dizo_amd.trainer.forward_wrap_with_option_len, the
reference's trainer.py:1446-1522) against the float64 brute-force oracle, on
a tiny random-init OPT on the CPU (no kernels involved)."""
import numpy as np
import pytest
import torch

from oracle import loss as OL


@pytest.fixture(scope="module")
def tiny_model():
    from transformers import OPTForCausalLM

    from dizo_amd.synth import SHAPES, opt_config

    torch.manual_seed(0)
    m = OPTForCausalLM(opt_config(SHAPES["opt-tiny"])).eval()
    return m


def _loop_mask(input_ids, option_len, pad_id):
    """The reference's own masking loop (trainer.py:1466-1475), for comparison."""
    shift_labels = torch.clone(input_ids)[..., 1:].contiguous()
    shift_labels[shift_labels == pad_id] = -100
    for _i, _len in enumerate(option_len):
        shift_labels[_i, :-_len] = -100
    return shift_labels


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_classification_loss_matches_bruteforce(tiny_model, seed):
    from dizo_amd.synth import PAD_ID, make_batch
    from dizo_amd.trainer import forward_wrap_with_option_len

    gen = torch.Generator().manual_seed(seed)
    b = make_batch(3, 512, gen=gen, min_len=5, max_len=12)
    if seed == 2:
        b["input_ids"][0, -3] = PAD_ID  # a pad-id collision inside a prompt
    with torch.no_grad():
        got = forward_wrap_with_option_len(tiny_model, **b, return_dict=True).loss
        logits = tiny_model(input_ids=b["input_ids"], attention_mask=b["attention_mask"]).logits
    want = OL.classification_loss(logits.double().numpy(), b["input_ids"].numpy(), b["labels"].tolist(),
                                  b["option_len"].tolist(), b["num_options"].tolist(), PAD_ID)
    assert float(got) == pytest.approx(want, rel=1e-5, abs=1e-6)


def test_multichoice_branch_matches_bruteforce(tiny_model):
    """Unequal num_options (the loop branch of trainer.py:1489-1500), option_len > 1."""
    from dizo_amd.synth import PAD_ID
    from dizo_amd.trainer import forward_wrap_with_option_len

    gen = torch.Generator().manual_seed(7)
    rows, L = 5, 16
    ids = torch.randint(2, 512, (rows, L), generator=gen)
    ids[1, :3] = PAD_ID
    mask = (ids != PAD_ID).long()
    b = {"input_ids": ids, "attention_mask": mask, "labels": torch.tensor([1, 1, 0, 0, 0]),
         "option_len": torch.tensor([2, 3, 1, 2, 4]), "num_options": torch.tensor([2, 2, 3, 3, 3])}
    with torch.no_grad():
        got = forward_wrap_with_option_len(tiny_model, **b, return_dict=True).loss
        logits = tiny_model(input_ids=ids, attention_mask=mask).logits
    want = OL.classification_loss(logits.double().numpy(), ids.numpy(), b["labels"].tolist(),
                                  b["option_len"].tolist(), b["num_options"].tolist(), PAD_ID)
    assert float(got) == pytest.approx(want, rel=1e-5, abs=1e-6)


def test_vectorised_option_mask_equals_reference_loop():
    gen = torch.Generator().manual_seed(3)
    for _ in range(20):
        rows, L = 6, int(torch.randint(4, 30, (1,), generator=gen))
        ids = torch.randint(0, 6, (rows, L), generator=gen)
        ol = torch.randint(1, L, (rows,), generator=gen)
        want = _loop_mask(ids, ol, 1)
        got = torch.clone(ids)[..., 1:].contiguous()
        got[got == 1] = -100
        pos = torch.arange(got.shape[1]).reshape(1, -1)
        got[pos < got.shape[1] - ol.reshape(-1, 1)] = -100
        assert torch.equal(got, want)


def test_bruteforce_closed_forms():
    """The oracle itself: uniform logits give log(2) per example; a decisive
    score gives ~0 loss; the pad id is never a target."""
    rows, L, V = 4, 5, 7
    ids = np.full((rows, L), 3)
    logits = np.zeros((rows, L, V))
    loss = OL.classification_loss(logits, ids, [0, 0, 1, 1], [1] * 4, [2] * 4, pad_id=1)
    assert loss == pytest.approx(np.log(2))
    logits[0, L - 2, 3] = 50.0  # candidate 0 of example 0 scores ~0, candidate 1 scores -log(7)
    loss = OL.classification_loss(logits, ids, [0, 0, 1, 1], [1] * 4, [2] * 4, pad_id=1)
    assert loss == pytest.approx((np.log(8 / 7) + np.log(2)) / 2, abs=1e-9)
    ids[2, L - 1] = 1  # pad-id target: row 2 has no option token
    assert np.isnan(OL.row_scores(logits, ids, [1] * 4, pad_id=1)[2])


def test_loss_without_kv_cache_is_identical(tiny_model):
    """The loss forward skips HF's key/value cache; the logits and the loss are unchanged."""
    from dizo_amd.synth import make_batch
    from dizo_amd.trainer import forward_wrap_with_option_len

    b = make_batch(4, 512, gen=torch.Generator().manual_seed(11), min_len=5, max_len=12)
    with torch.no_grad():
        a = forward_wrap_with_option_len(tiny_model, **b, return_dict=True).loss
        c = forward_wrap_with_option_len(tiny_model, **b, use_cache=True, return_dict=True).loss
        la = tiny_model(input_ids=b["input_ids"], attention_mask=b["attention_mask"], use_cache=False).logits
        lc = tiny_model(input_ids=b["input_ids"], attention_mask=b["attention_mask"], use_cache=True).logits
    assert torch.equal(a, c)
    assert torch.equal(la, lc)
