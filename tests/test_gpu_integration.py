"""The drop-in as a maintainer would wire it: ZOTrainerMixin mixed into a
transformers.Trainer subclass (the reference's OurTrainer), arguments from a
TrainingArguments subclass carrying the ZO fields (the reference's
OurArguments), and the ZO branch of the reference's training loop
(trainer.py:1206-1326 with gradient_accumulation_steps 1) calling zo_step and
zo_update. It must give the weights and losses of ZOTrainer bit for bit,
across a DiZO event."""
from dataclasses import dataclass
from typing import Optional

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().view({2: torch.int16, 4: torch.int32}[t.element_size()])


def _classes():
    from transformers import Trainer, TrainingArguments

    from dizo_amd.trainer import ZOTrainerMixin

    @dataclass
    class OurArguments(TrainingArguments):
        # the fields of run.py:35-118 that the ZO path reads
        trainer: str = "zo"
        zo_eps: float = 1e-3
        enhanced: Optional[str] = None
        non_diff: bool = False

    class OurTrainer(ZOTrainerMixin, Trainer):
        """trainer.py's OurTrainer with zo_perturb_parameters / zo_forward / zo_step /
        zo_update / forward_wrap_with_option_len taken from the mixin."""

    return OurArguments, OurTrainer


@pytest.mark.parametrize("enhanced", [None, "zo"])
def test_mixin_in_hf_trainer_matches_zotrainer(enhanced, tmp_path):
    from dizo_amd.synth import Cycle, build_opt, make_batches
    from dizo_amd.trainer import ZOArguments, ZOTrainer
    OurArguments, OurTrainer = _classes()
    steps, lr = 55, 1e-3
    batches = make_batches(5, 4, 512, seed=71, device="cuda", min_len=8, max_len=20)

    model_a = build_opt("opt-tiny", torch.float16, "cuda", seed=7)
    model_b = build_opt("opt-tiny", torch.float16, "cuda", seed=7)
    np.random.seed(26)
    ref = ZOTrainer(model_a, ZOArguments(learning_rate=lr, zo_eps=1e-3, max_steps=steps, enhanced=enhanced),
                    train_dataloader=Cycle(batches))
    want = [float(ref.training_step(batches[k % 5])) for k in range(steps)]
    ref.zo_close()

    args = OurArguments(output_dir=str(tmp_path), learning_rate=lr, max_steps=steps, report_to=[],
                        enhanced=enhanced, zo_eps=1e-3)
    tr = OurTrainer(model=model_b, args=args)
    # trainer.py:1099-1101 and 1147-1171 (scheduler, trainable set, anchor, DiZO), as one call
    tr.zo_setup(model_b, Cycle(batches), optimizer=tr.create_optimizer())
    np.random.seed(26)
    got = []
    tr_loss = torch.tensor(0.0, device="cuda")
    for step in range(steps):  # trainer.py:1206-1326, the ZO branch
        inputs = batches[step % 5]
        tr_loss_step = tr.zo_step(model_b, inputs)
        tr_loss += tr_loss_step
        tr.zo_update(tr.args, model_b)
        tr.state.global_step += 1
        got.append(float(tr_loss_step))
    tr.zo_flush()
    torch.cuda.synchronize()
    assert got == want
    for (n, a), (_, b) in zip(model_a.named_parameters(), model_b.named_parameters()):
        assert torch.equal(_bits(a.data), _bits(b.data)), n
    tr.zo_close()
