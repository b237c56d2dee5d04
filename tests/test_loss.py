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


def test_option_mask_equals_reference_loop():
    """shift_option_labels sets exactly the elements of the reference's loop,
    option_len 0 (nothing masked) and longer than the row included; with a
    window, the loop leaves nothing unmasked before it and the window's
    columns are the loop's last ones."""
    from dizo_amd.trainer import option_window, shift_option_labels

    gen = torch.Generator().manual_seed(3)
    windows = 0
    for it in range(60):
        rows, L = 6, int(torch.randint(2, 30, (1,), generator=gen))
        ids = torch.randint(0, 6, (rows, L), generator=gen)
        hi = L + 2 if it % 3 == 0 else max(2, L // 3)
        ol = torch.randint(0 if it % 4 == 0 else 1, hi, (rows,), generator=gen)
        want = _loop_mask(ids, ol, 1)
        assert torch.equal(shift_option_labels(ids, ol, 1), want)
        w = option_window(ol.tolist(), L)
        if w is None:
            assert int(ol.min()) == 0 or int(ol.max()) + 1 >= L
            continue
        windows += 1
        assert bool((want[:, :L - w] == -100).all())
        assert torch.equal(shift_option_labels(ids, ol, 1, window=w), want[:, L - w:])
    assert windows >= 10


def test_option_window_edges():
    from dizo_amd.trainer import option_window

    assert option_window([1, 1, 1], 128) == 2
    assert option_window([1, 3, 2], 10) == 4
    assert option_window([1, 0, 2], 10) is None  # [:-0] keeps the whole row
    assert option_window([9], 10) is None         # the window is the whole sequence
    assert option_window([], 10) is None


@pytest.mark.parametrize("case", ["padded", "multichoice", "zero_len"])
def test_option_head_loss_equals_full_loss(tiny_model, case):
    """The option-position head (logits only for the last max(option_len) + 1
    positions) gives the full-logit loss; in float64 the only difference is
    the LM head's row count, so they agree to ~1e-12. The float64
    brute-force oracle pins both."""
    from dizo_amd.synth import PAD_ID, make_batch
    from dizo_amd.trainer import option_len_loss

    m64 = tiny_model.double()
    try:
        gen = torch.Generator().manual_seed(21)
        if case == "padded":
            b = make_batch(4, 512, gen=gen, min_len=5, max_len=14)
            b["input_ids"][1, -4] = PAD_ID
        else:
            rows, L = 5, 16
            ids = torch.randint(2, 512, (rows, L), generator=gen)
            ids[1, :3] = PAD_ID
            ol = [2, 3, 1, 2, 4] if case == "multichoice" else [2, 0, 1, 2, 1]
            b = {"input_ids": ids, "attention_mask": (ids != PAD_ID).long(),
                 "labels": torch.tensor([1, 1, 0, 0, 0]), "option_len": torch.tensor(ol),
                 "num_options": torch.tensor([2, 2, 3, 3, 3])}
        with torch.no_grad():
            full = option_len_loss(m64, False, **b, return_dict=True).loss
            m64.dz_option_head = True
            head = option_len_loss(m64, False, **b, return_dict=True).loss
            logits = m64(input_ids=b["input_ids"], attention_mask=b["attention_mask"]).logits
        want = OL.classification_loss(logits.numpy(), b["input_ids"].numpy(), b["labels"].tolist(),
                                      b["option_len"].tolist(), b["num_options"].tolist(), PAD_ID)
        assert float(full) == pytest.approx(want, rel=1e-10, abs=1e-12)
        assert float(head) == pytest.approx(float(full), rel=1e-10, abs=1e-12)
    finally:
        m64.dz_option_head = False
        m64.float()


def test_option_head_asks_for_the_window_only(tiny_model):
    """With the option head the forward is asked for the logits of the last
    max(option_len) + 1 positions (as index positions), not the whole sequence."""
    from dizo_amd.synth import make_batch
    from dizo_amd.trainer import option_len_loss

    b = make_batch(2, 512, gen=torch.Generator().manual_seed(5), min_len=20, max_len=24)
    b["option_len"] = torch.tensor([1, 2, 1, 3])
    seen = {}
    orig = tiny_model.forward

    def spy(*a, **kw):
        seen.update(kw)
        return orig(*a, **kw)

    tiny_model.forward = spy
    try:
        tiny_model.dz_option_head = True
        with torch.no_grad():
            out = option_len_loss(tiny_model, False, **b)
        L = b["input_ids"].shape[1]
        assert torch.equal(seen["logits_to_keep"], torch.arange(L - 4, L))
        assert out[1].shape[1] == 4
    finally:
        tiny_model.dz_option_head = False
        del tiny_model.forward


def test_host_ints_reads_a_tensor_once_per_version():
    from dizo_amd.trainer import host_ints

    t = torch.tensor([2, 2, 3])
    assert host_ints(t) == [2, 2, 3]
    assert host_ints([1, 2]) == [1, 2]
    t[0] = 5
    assert host_ints(t) == [5, 2, 3]


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


def test_llama_without_pad_id_matches_bruteforce():
    """Another model family through the same forward (the reference loads any
    causal LM, run.py:157-181): a tiny random-init LLaMA whose config has no
    pad id. The reference's `labels == None` masks nothing; so does the
    library. Full logits and the option-position window, against the
    brute-force oracle."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from dizo_amd.synth import make_batch
    from dizo_amd.trainer import forward_wrap_with_option_len

    torch.manual_seed(3)
    cfg = LlamaConfig(vocab_size=512, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
                      pad_token_id=None)
    m = LlamaForCausalLM(cfg).eval()
    assert m.config.pad_token_id is None
    gen = torch.Generator().manual_seed(11)
    b = make_batch(3, 512, gen=gen, min_len=5, max_len=12)
    b["attention_mask"] = torch.ones_like(b["input_ids"])  # no padding in this family's batches
    with torch.no_grad():
        full = forward_wrap_with_option_len(m, **b, return_dict=True).loss
        logits = m(input_ids=b["input_ids"], attention_mask=b["attention_mask"]).logits
        m.dz_option_head = True
        head = forward_wrap_with_option_len(m, **b, return_dict=True).loss
        m.dz_option_head = False
    want = OL.classification_loss(logits.double().numpy(), b["input_ids"].numpy(), b["labels"].tolist(),
                                  b["option_len"].tolist(), b["num_options"].tolist(), None)
    assert float(full) == pytest.approx(want, rel=1e-5, abs=1e-6)
    assert float(head) == pytest.approx(want, rel=1e-5, abs=1e-6)


@pytest.mark.parametrize("seed", [0, 3])
def test_reference_forward_loss_restatement_matches_bruteforce(tiny_model, seed):
    """oracle.ref_torch.forward_loss (the CPU baseline's forward: full logits and
    the reference's own per-row masking loop, trainer.py:1446-1522) against the
    float64 brute force."""
    from dizo_amd.synth import PAD_ID, make_batch
    from oracle import ref_torch as R

    b = make_batch(3, 512, gen=torch.Generator().manual_seed(seed), min_len=5, max_len=12)
    if seed == 3:
        b["input_ids"][1, -4] = PAD_ID
    with torch.no_grad():
        got = R.forward_loss(tiny_model, pad_id=PAD_ID, **b)
        logits = tiny_model(input_ids=b["input_ids"], attention_mask=b["attention_mask"]).logits
    want = OL.classification_loss(logits.double().numpy(), b["input_ids"].numpy(), b["labels"].tolist(),
                                  b["option_len"].tolist(), b["num_options"].tolist(), PAD_ID)
    assert float(got) == pytest.approx(want, rel=1e-5, abs=1e-6)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_reference_apply_ratio_matches_arith(dt):
    """oracle.ref_torch.apply_ratio (trainer.py:428-436 with the ratio supplied)
    against oracle.arith.apply with alpha rounded to the dtype, and alpha = 1
    leaving R(R(theta - theta0) + theta0)."""
    from oracle import arith as A
    from oracle import ref_torch as R

    name = {torch.float16: A.F16, torch.bfloat16: A.BF16, torch.float32: A.F32}[dt]
    view = torch.int32 if dt == torch.float32 else torch.int16
    gen = torch.Generator().manual_seed(2)
    th = (torch.randn(4099, generator=gen) * 0.02).to(dt)
    t0 = (th.float() + 1e-3 * torch.randn(4099, generator=gen)).to(dt)
    for a in (0.9, 1.0):
        p = [th.clone()]
        R.apply_ratio(p, [t0], torch.tensor(a, dtype=dt))
        bits = lambda x: x.view(view).numpy().view(np.uint32 if dt == torch.float32 else np.uint16)  # noqa: E731
        alpha_bits = bits(torch.tensor([a], dtype=dt))
        want = A.apply(bits(th), bits(t0), np.repeat(alpha_bits, th.numel()), name)
        np.testing.assert_array_equal(bits(p[0]), want)
