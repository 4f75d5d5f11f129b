"""The training step's host logic on the CPU: micro-batch splitting, the
schedules' backward order
and loss scaling (pipeline_parallel/schedules/gpipe.py, one_f_one_b.py,
base.py:111-126), and the token-weighted loss metric (training/metrics.py:
68-121), checked on a small CPU model against closed forms."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch
from torch import nn

import nano_megatron_amd as nm
from nano_megatron_amd.train import _microbatches


def _rows(batch, size):
    """The micro-batches the step should see: consecutive row ranges."""
    n = batch["input_ids"].size(0) // size
    return [{k: v[i * size:(i + 1) * size] for k, v in batch.items()} for i in range(n)]


def test_microbatches_are_row_views_and_pass_other_entries() -> None:
    ids = torch.arange(24).reshape(6, 4)
    batch = {"input_ids": ids, "labels": ids + 1, "position_ids": torch.arange(4)[None], "scale": 2.0}
    parts = _microbatches(batch, 2)
    assert len(parts) == 3
    for i, part in enumerate(parts):
        assert torch.equal(part["input_ids"], ids[2 * i:2 * i + 2])
        assert torch.equal(part["labels"], ids[2 * i:2 * i + 2] + 1)
        assert part["position_ids"] is batch["position_ids"] and part["scale"] == 2.0
        assert part["input_ids"].data_ptr() == ids[2 * i].data_ptr()  # views, no copies


@pytest.mark.parametrize("batch,mbs,match", [
    ({"input_ids": torch.zeros(4, 2)}, 0, "does not split"),
    ({"input_ids": torch.zeros(4, 2)}, 3, "does not split"),
    ({"input_ids": torch.zeros(4, 2), "labels": torch.zeros(5, 2)}, 2, "labels has 5 rows"),
])
def test_microbatches_reject_uneven_batches(batch, mbs, match) -> None:
    with pytest.raises(ValueError, match=match):
        _microbatches(batch, mbs)


class TinyLM(nn.Module):
    """Embedding + linear head with a mean token cross-entropy (ignore -100), in
    fp64 so that the order of the gradient additions stays below the
    tolerances: enough to exercise the step's host logic on the CPU."""

    def __init__(self) -> None:
        super().__init__()
        torch.manual_seed(0)
        self.emb = nn.Embedding(11, 8, dtype=torch.float64)
        self.head = nn.Linear(8, 11, dtype=torch.float64)
        self.calls: list[int] = []

    def forward(self, input_ids, *, labels=None, position_ids=None, microbatch_index=0):
        self.calls.append(microbatch_index)
        logits = self.head(self.emb(input_ids))
        loss = nn.functional.cross_entropy(logits.reshape(-1, 11), labels.reshape(-1), ignore_index=-100)
        return SimpleNamespace(loss=loss)


def _batch():
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 11, (6, 5), generator=g)
    labels = torch.randint(0, 11, (6, 5), generator=g)
    labels[0, :4] = -100  # uneven token counts per micro-batch
    labels[3, :2] = -100
    return {"input_ids": ids, "labels": labels}


@pytest.mark.parametrize("schedule", ["gpipe", "1f1b"])
def test_train_step_accumulates_the_mean_of_microbatch_losses(schedule) -> None:
    """Gradient = d/dw of the mean over micro-batches of each micro-batch's
    mean loss (the schedules divide each by their number); the reported loss
    is the token-weighted mean; micro-batches are numbered from step x
    accumulation steps; the step applies clip and the optimizer."""
    batch = _batch()
    model = TinyLM()
    ref = TinyLM()
    opt = torch.optim.SGD(model.parameters(), lr=0.1)
    out = nm.train_step(model, opt, batch, micro_batch_size=2, gradient_accumulation_steps=3,
                        schedule=schedule, clip_grad_norm=None, step_index=4)
    assert model.calls == [12, 13, 14]
    parts = _rows(batch, 2)
    losses = [ref(p["input_ids"], labels=p["labels"]).loss for p in parts]
    (sum(losses) / 3).backward()
    with torch.no_grad():
        for p in ref.parameters():
            p -= 0.1 * p.grad
    for a, b in zip(model.parameters(), ref.parameters()):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
    tokens = [(p["labels"] != -100).sum().item() for p in parts]
    weighted = sum(float(l.detach()) * t for l, t in zip(losses, tokens)) / sum(tokens)
    assert out.metrics["token_count"] == sum(tokens)
    assert out.metrics["loss"] == pytest.approx(weighted, rel=1e-12)
    assert out.metrics["learning_rate"] == pytest.approx(0.1)
    assert float(out.loss) == pytest.approx(float(sum(losses).detach() / 3), rel=1e-12)


def test_train_step_backward_order_per_schedule() -> None:
    """GPipe runs every forward, then the backwards newest first; 1F1B at one
    stage alternates forward and backward."""
    order: list[str] = []

    class Probe(TinyLM):
        def forward(self, input_ids, *, labels=None, position_ids=None, microbatch_index=0):
            out = super().forward(input_ids, labels=labels, microbatch_index=microbatch_index)
            order.append(f"F{microbatch_index}")
            out.loss.register_hook(lambda g, i=microbatch_index: order.append(f"B{i}"))
            return out

    for schedule, expected in (("gpipe", ["F0", "F1", "F2", "B2", "B1", "B0"]),
                               ("1f1b", ["F0", "B0", "F1", "B1", "F2", "B2"])):
        order.clear()
        model = Probe()
        nm.train_step(model, torch.optim.SGD(model.parameters(), lr=0.0), _batch(), micro_batch_size=2,
                      schedule=schedule, clip_grad_norm=None)
        assert order == expected, schedule


def test_train_step_clips_and_follows_the_lr_scheduler() -> None:
    class Sched:
        def __init__(self) -> None:
            self.learning_rate = 0.05
            self.completed = None

        def set_completed_steps(self, n: int) -> None:
            self.completed = n

    model, ref = TinyLM(), TinyLM()
    sched = Sched()
    opt = torch.optim.SGD(model.parameters(), lr=123.0)
    out = nm.train_step(model, opt, _batch(), micro_batch_size=3, schedule="gpipe", clip_grad_norm=0.01,
                        lr_scheduler=sched, step_index=7)
    assert sched.completed == 8 and out.metrics["learning_rate"] == 0.05
    parts = _rows(_batch(), 3)
    (sum(ref(p["input_ids"], labels=p["labels"]).loss for p in parts) / 2).backward()
    norm = torch.nn.utils.clip_grad_norm_(ref.parameters(), 0.01)
    assert out.metrics["grad_norm"] == pytest.approx(float(norm), rel=1e-12)
    with torch.no_grad():
        for p in ref.parameters():
            p -= 0.05 * p.grad
    for a, b in zip(model.parameters(), ref.parameters()):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)


def test_train_step_rejects_bad_arguments() -> None:
    model = TinyLM()
    opt = torch.optim.SGD(model.parameters(), lr=0.1)
    with pytest.raises(ValueError, match="gradient_accumulation_steps is 2"):
        nm.train_step(model, opt, _batch(), micro_batch_size=2, gradient_accumulation_steps=2)
    with pytest.raises(ValueError, match="unknown schedule"):
        nm.train_step(model, opt, _batch(), micro_batch_size=2, schedule="interleaved")
    with pytest.raises(ValueError, match="labels"):
        nm.train_step(model, opt, {"input_ids": torch.zeros(2, 3, dtype=torch.long)}, micro_batch_size=1)
