"""The training step captured as a HIP graph (CapturedTrainStep) against eager
steps: replays give the eager losses, parameters and optimizer state bit for
bit, with eager work and a synchronisation between replays; out-of-range
targets raise before any update, as in the eager forward."""

from __future__ import annotations

import pytest
import torch

import nano_megatron_amd as nm
from nano_megatron_amd.graph import CapturedTrainStep
from nano_megatron_amd.optim import MasterAdamW

pytestmark = pytest.mark.gpu

VOCAB = 1024


def small_model(device, mode: str, offload: bool = False, layers: int = 2, block_interval: int = 1):
    cfg = nm.GPTConfig(layers=layers, hidden_size=256, ffn_hidden_size=688, heads=4, seq_length=128,
                       vocab_size=VOCAB, norm_epsilon=1e-5, rope_theta=1e4)
    ck = nm.ActivationCheckpointConfig(mode=mode, offload_saved_tensors=offload, block_interval=block_interval)
    torch.manual_seed(0)
    return nm.GPTModel(cfg, activation_checkpoint_config=ck).to(device=device, dtype=torch.bfloat16).train()


def batches(device, n: int):
    g = torch.Generator(device=device).manual_seed(7)
    out = []
    for _ in range(n):
        ids = torch.randint(0, VOCAB, (2, 129), device=device, generator=g)
        out.append((ids[:, :128].contiguous(), ids[:, 1:].contiguous()))
    return out


def optimizer(model):
    return MasterAdamW(model.parameters(), lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                       clip_grad_norm=1.0)


@pytest.mark.parametrize("mode", ["full", "none", "selective"])
def test_captured_step_replays_match_eager_steps(device, mode) -> None:
    data = batches(device, 4)
    eager = small_model(device, mode)
    opt_e = optimizer(eager)
    losses_e = []
    for x, y in data:
        opt_e.zero_grad()
        loss = eager(x, labels=y).loss
        loss.backward()
        opt_e.step()
        losses_e.append(loss.detach().clone())

    model = small_model(device, mode)
    opt = optimizer(model)
    cap = CapturedTrainStep(model, opt, data[0][0], data[0][1])
    losses_g = []
    for x, y in data:
        losses_g.append(cap.step(x, y).clone())
        # the program's own work and a synchronisation between replays
        a = torch.randn(256, 256, device=device)
        (a @ a).sum().item()
        torch.cuda.synchronize()

    for i, (le, lg) in enumerate(zip(losses_e, losses_g)):
        assert torch.isfinite(le) and torch.equal(le, lg), f"step {i}: {le.item()} vs {lg.item()}"
    assert opt.step_count == opt_e.step_count == len(data)
    for (name, p), q in zip(eager.named_parameters(), model.parameters()):
        assert torch.equal(p, q), name
    for attr in ("master", "exp_avg", "exp_avg_sq"):
        assert torch.equal(getattr(opt_e, attr), getattr(opt, attr)), attr
    assert torch.equal(opt_e.last_grad_norm, opt.last_grad_norm)


def test_captured_steps_on_the_same_batch_match_eager_steps(device) -> None:
    """Replays on the captured batch (no new labels: no check, no host wait
    between them, the optimizer's step scalars staged through alternating host
    records) give the eager steps' parameters and optimizer state bit for bit."""
    (x, y), = batches(device, 1)
    eager = small_model(device, "full")
    opt_e = optimizer(eager)
    for _ in range(5):
        opt_e.zero_grad()
        eager(x, labels=y).loss.backward()
        opt_e.step()
    model = small_model(device, "full")
    opt = optimizer(model)
    cap = CapturedTrainStep(model, opt, x, y)
    for _ in range(5):
        cap.step()
    torch.cuda.synchronize()
    assert opt.step_count == opt_e.step_count == 5
    for (name, p), q in zip(eager.named_parameters(), model.parameters()):
        assert torch.equal(p, q), name
    for attr in ("master", "exp_avg", "exp_avg_sq"):
        assert torch.equal(getattr(opt_e, attr), getattr(opt, attr)), attr


@pytest.mark.parametrize("block_interval", [1, 2])
def test_captured_step_prefetches_recompute(device, monkeypatch, block_interval) -> None:
    """A captured full-recompute step starts each checkpointed block's recompute
    during the backward of the checkpointed block after it (one prefetch per
    checkpointed block but the last in forward order, none in an eager step),
    and its replays still give the eager steps' parameters bit for bit, with
    checkpointed and eager blocks alternating (block_interval 2) too."""
    from nano_megatron_amd import block as B

    calls = []
    orig = B._prefetch_recompute
    monkeypatch.setattr(B, "_prefetch_recompute", lambda ctx, dev: (calls.append(1), orig(ctx, dev)))
    layers = 4
    checkpointed = len(range(0, layers, block_interval))
    data = batches(device, 3)
    eager = small_model(device, "full", layers=layers, block_interval=block_interval)
    opt_e = optimizer(eager)
    for x, y in data:
        opt_e.zero_grad()
        eager(x, labels=y).loss.backward()
        opt_e.step()
    assert not calls

    model = small_model(device, "full", layers=layers, block_interval=block_interval)
    opt = optimizer(model)
    cap = CapturedTrainStep(model, opt, data[0][0], data[0][1])
    assert len(calls) == checkpointed - 1
    for x, y in data:
        cap.step(x, y)
    torch.cuda.synchronize()
    for (name, p), q in zip(eager.named_parameters(), model.parameters()):
        assert torch.equal(p, q), name


def test_captured_step_rejects_out_of_range_labels(device) -> None:
    (x, y), = batches(device, 1)
    model = small_model(device, "full")
    opt = optimizer(model)
    cap = CapturedTrainStep(model, opt, x, y)
    before = [p.detach().clone() for p in model.parameters()]
    bad = y.clone()
    bad[1, 5] = VOCAB
    with pytest.raises(ValueError, match="outside"):
        cap.step(x, bad)
    # the captured labels buffer now holds the rejected targets: a step without
    # new labels checks them again instead of replaying
    with pytest.raises(ValueError, match="outside"):
        cap.step()
    torch.cuda.synchronize()
    assert opt.step_count == 0
    for a, p in zip(before, model.parameters()):
        assert torch.equal(a, p)
    # a valid batch afterwards still steps
    loss = cap.step(x, y)
    assert torch.isfinite(loss) and opt.step_count == 1


def test_captured_step_refuses_offload_and_shape_changes(device) -> None:
    (x, y), = batches(device, 1)
    model = small_model(device, "full", offload=True)
    with pytest.raises(ValueError, match="offload_saved_tensors"):
        CapturedTrainStep(model, optimizer(model), x, y)
    # a layer outside the fused block (biases) recomputes under torch's checkpoint
    cfg = nm.GPTConfig(layers=1, hidden_size=256, ffn_hidden_size=688, heads=4, seq_length=128,
                       vocab_size=VOCAB, bias=True)
    for mode in ("full", "selective"):
        torch.manual_seed(0)
        biased = nm.GPTModel(cfg, activation_checkpoint_config=nm.ActivationCheckpointConfig(mode=mode))
        biased = biased.to(device=device, dtype=torch.bfloat16).train()
        with pytest.raises(ValueError, match="torch.utils.checkpoint"):
            CapturedTrainStep(biased, optimizer(biased), x, y)
    model = small_model(device, "full")
    cap = CapturedTrainStep(model, optimizer(model), x, y)
    with pytest.raises(ValueError, match="shape"):
        cap.step(x[:1], y[:1])
