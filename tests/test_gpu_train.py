"""The training step with gradient accumulation on the GPU against the oracle
model stepped the reference's way (training/trainer.py:424-474: micro-batch
losses divided by their number, backwards in the schedule's order, clip,
AdamW): fp32 at rtol 1e-5, bf16 with the fp32-master optimizer at the bf16
tolerances."""

from __future__ import annotations

import pytest
import torch

import nano_megatron_amd as nm
from nano_megatron_amd.optim import MasterAdamW
from oracle import reference as R
from parity import assert_bf16_grads, assert_close_scaled, loss_rtol

from test_gpu_dropout import ForkRNG

pytestmark = pytest.mark.gpu


def config(**kw):
    base = dict(layers=2, hidden_size=256, ffn_hidden_size=688, heads=4, seq_length=128, vocab_size=8192,
                norm_epsilon=1e-5, rope_theta=1e4)
    base.update(kw)
    return nm.GPTConfig(**base)


def batch(n=4, seq=128, vocab=8192):
    g = torch.Generator().manual_seed(21)
    ids = torch.randint(0, vocab, (n, seq + 1), generator=g)
    labels = ids[:, 1:].clone()
    labels[1, :40] = -100  # micro-batches with different token counts
    return {"input_ids": ids[:, :seq].contiguous(), "labels": labels}


def pair(cfg, dtype, device, mode="full"):
    ck = nm.ActivationCheckpointConfig(mode=mode)
    torch.manual_seed(0)
    ours = nm.GPTModel(cfg, activation_checkpoint_config=ck).to(device=device, dtype=dtype)
    torch.manual_seed(0)
    ref = R.OracleGPTModel(cfg, activation_checkpoint_config=ck).to(dtype=dtype)
    ref.load_state_dict({k: v.cpu() for k, v in ours.state_dict().items()})
    return ours, ref


def oracle_accumulate(ref, b, micro, schedule):
    """The schedule at one stage: each micro-batch loss / n, backwards newest
    first (GPipe) or right after each forward (1F1B); returns the token-weighted loss."""
    parts = [{k: v[i:i + micro] for k, v in b.items()} for i in range(0, b["input_ids"].size(0), micro)]
    n = len(parts)
    losses = []
    for p in parts:
        losses.append(ref(p["input_ids"], labels=p["labels"]).loss)
        if schedule == "1f1b":
            (losses[-1] / n).backward()
    if schedule == "gpipe":
        for loss in reversed(losses):
            (loss / n).backward()
    tokens = [float((p["labels"] != -100).sum()) for p in parts]
    return sum(float(l.detach()) * t for l, t in zip(losses, tokens)) / sum(tokens)


def test_fp32_accumulated_step_matches_oracle(device) -> None:
    """Four sequences as two micro-batches, full recompute, torch AdamW with
    clip 1.0 (the fp32 configuration's optimizer, data_parallel/_common.py:
    242-252): loss, gradient norm, every accumulated gradient, and the weights
    after the step."""
    ours, ref = pair(config(), torch.float32, device)
    b = batch()
    opt = torch.optim.AdamW(ours.parameters(), lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    out = nm.train_step(ours, opt, {k: v.to(device) for k, v in b.items()}, micro_batch_size=2,
                        gradient_accumulation_steps=2, schedule="gpipe", clip_grad_norm=1.0)
    ref.train()
    ropt = torch.optim.AdamW(ref.parameters(), lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    loss = oracle_accumulate(ref, b, 2, "gpipe")
    # torch's clip (ddp.py:108-117) with the norm in fp64: torch's fp32 CPU norm
    # of the 2M-element embedding gradient is off by ~1e-4 (its summation order)
    norm = torch.sqrt(sum(p.grad.double().square().sum() for p in ref.parameters()))
    coef = R.clip_coefficient(norm.float(), 1.0)
    for p in ref.parameters():
        p.grad.mul_(coef)
    ropt.step()
    assert out.metrics["loss"] == pytest.approx(loss, rel=1e-5)
    assert out.metrics["grad_norm"] == pytest.approx(float(norm), rel=1e-5)
    assert out.metrics["token_count"] == float((b["labels"] != -100).sum())
    theirs = dict(ref.named_parameters())
    for name, p in ours.named_parameters():
        q = theirs[name]
        # the accumulated, clipped gradients (left in .grad by the step)
        assert_close_scaled(p.grad, q.grad, torch.float32, msg=name)
        # the first AdamW step is ~lr * sign(grad): the weights where the
        # gradient stands clear of its rounding noise
        clear = q.grad.abs() > 1e-3 * q.grad.abs().max()
        torch.testing.assert_close(p.detach().cpu()[clear], q.detach()[clear], rtol=1e-5, atol=1e-6, msg=name)


@pytest.mark.parametrize("schedule", ["gpipe", "1f1b"])
def test_bf16_master_adamw_accumulated_step_matches_oracle(device, schedule) -> None:
    """bf16 parameters, gradients accumulated in bf16 in the schedule's order,
    the fp32-master AdamW with clip (data_parallel/_zero.py:130-199): loss,
    gradient norm and the fp32 master after the step."""
    cfg = config(kv_heads=2)
    ours, ref = pair(cfg, torch.bfloat16, device)
    b = batch()
    opt = MasterAdamW(ours.parameters(), lr=1e-3, weight_decay=0.1, clip_grad_norm=1.0)
    init = opt.master.cpu().clone()
    out = nm.train_step(ours, opt, {k: v.to(device) for k, v in b.items()}, micro_batch_size=1,
                        schedule=schedule)
    ref.train()
    loss = oracle_accumulate(ref, b, 1, schedule)
    # the accumulated bf16 gradients (left in .grad by the step) against the
    # oracle's, both measured against the fp32 oracle accumulated the same way
    twin = R.OracleGPTModel(cfg).train()
    twin.load_state_dict({k: v.float() for k, v in ref.state_dict().items()})
    oracle_accumulate(twin, b, 1, schedule)
    assert_bf16_grads(ours, ref, twin)
    grads = torch.cat([p.grad.float().reshape(-1) for p in ref.parameters()])
    norm = grads.norm()
    coef = R.clip_coefficient(norm, 1.0)
    master = init.clone()
    m, v = torch.zeros_like(master), torch.zeros_like(master)
    R.adamw_master_step(master, m, v, grads * coef, step=1, lr=1e-3, weight_decay=0.1)
    assert out.metrics["loss"] == pytest.approx(loss, rel=loss_rtol(torch.bfloat16))
    assert out.metrics["grad_norm"] == pytest.approx(float(norm), rel=2e-2)
    # the first AdamW step moves each weight by about lr * sign(grad): compare
    # the step taken, where the oracle's gradient is clearly non-zero
    moved, expected = opt.master.cpu() - init, master - init
    clear = grads.abs() > 1e-2 * grads.abs().max()
    assert float(clear.float().mean()) > 0.05
    torch.testing.assert_close(moved[clear], expected[clear], rtol=0.0, atol=2e-4)


def test_one_microbatch_step_equals_the_plain_step(device) -> None:
    """With one micro-batch the step is forward, backward and the optimizer,
    bit for bit."""
    cfg = config()
    b = {k: v.to(device) for k, v in batch(n=2).items()}
    results = []
    for use_step in (True, False):
        torch.manual_seed(0)
        model = nm.GPTModel(cfg, activation_checkpoint_config=nm.ActivationCheckpointConfig(mode="full"))
        model = model.to(device=device, dtype=torch.bfloat16).train()
        opt = MasterAdamW(model.parameters(), lr=1e-3)
        if use_step:
            out = nm.train_step(model, opt, b, micro_batch_size=2)
            loss = out.loss
        else:
            opt.zero_grad()
            loss = model(b["input_ids"], labels=b["labels"]).loss
            loss.backward()
            opt.step()
        results.append((loss.detach().clone(), opt.master.clone()))
    assert torch.equal(results[0][0], results[1][0])
    assert torch.equal(results[0][1], results[1][1])


def test_microbatch_index_keys_the_dropout_streams(device) -> None:
    """Two identical sequences as two micro-batches: with dropout and a forked
    RNG their masks differ (the index is part of the stream key,
    trainer.py:103-113), without dropout their losses are equal."""
    seq = torch.randint(0, 8192, (1, 129), generator=torch.Generator().manual_seed(3))
    b = {"input_ids": seq[:, :128].repeat(2, 1).to(device), "labels": seq[:, 1:].repeat(2, 1).to(device)}
    for p, differ in ((0.1, True), (0.0, False)):
        torch.manual_seed(0)
        model = nm.GPTModel(config(dropout=p), rng=ForkRNG(5)).to(device=device, dtype=torch.bfloat16)
        opt = MasterAdamW(model.parameters(), lr=0.0, weight_decay=0.0)
        out = nm.train_step(model, opt, b, micro_batch_size=1, schedule="1f1b")
        a, c = (float(x.detach()) for x in out.losses)
        assert (a != c) == differ


def test_master_adamw_resumes_from_its_state_dict(device) -> None:
    """Two steps, save (model and optimizer), a third step; a fresh model and
    optimizer loaded from the saved state take the same third step, bit for
    bit (data_parallel/_zero.py:234-301)."""
    cfg = config(layers=1)
    b = {k: v.to(device) for k, v in batch(n=2).items()}

    def fresh():
        torch.manual_seed(0)
        m = nm.GPTModel(cfg).to(device=device, dtype=torch.bfloat16)
        return m, MasterAdamW(m.parameters(), lr=1e-3)

    model, opt = fresh()
    for step in range(2):
        nm.train_step(model, opt, b, micro_batch_size=2, step_index=step)
    saved_model = {k: v.clone() for k, v in model.state_dict().items()}
    saved_opt = opt.state_dict()
    third = nm.train_step(model, opt, b, micro_batch_size=2, step_index=2)
    model2, opt2 = fresh()
    model2.load_state_dict(saved_model)
    opt2.load_state_dict(saved_opt)
    again = nm.train_step(model2, opt2, b, micro_batch_size=2, step_index=2)
    assert torch.equal(third.loss, again.loss)
    assert torch.equal(opt.master, opt2.master) and torch.equal(opt.exp_avg_sq, opt2.exp_avg_sq)
    assert opt2.step_count == 3
    bad = dict(saved_opt, numels=saved_opt["numels"][:-1])
    with pytest.raises(ValueError, match="layout changed"):
        opt2.load_state_dict(bad)
