"""The parity bars of tests/parity.py can fail: on the CPU, with the oracle's
own gradients planted with the mistakes a broken kernel would make (a zeroed
gradient, one scaled by 1.05 or 0.95), each bar rejects them, while it
accepts the oracle's bf16 gradients themselves and with one bf16 ulp of noise
per element.  The mistakes are planted in copies of the oracle's outputs, on
the CPU; nothing here runs a kernel."""

from __future__ import annotations

import math

import pytest
import torch

import nano_megatron_amd as nm
from oracle import reference as R
from parity import (
    BF16_GRAD_MAX_REF_ERR,
    assert_close_scaled,
    assert_loss_close,
    bf16_grad_error,
    close_scaled,
    loss_rtol,
)


def _oracle_grads(cfg, batch, seq, seed=1234):
    """Loss and gradients of the oracle in bf16 and of its fp32 twin on the
    same bf16 weights, seeded uniform tokens."""
    torch.manual_seed(seed)
    none = nm.ActivationCheckpointConfig(mode="none")
    ref = R.OracleGPTModel(cfg, activation_checkpoint_config=none).to(dtype=torch.bfloat16)
    ref32 = R.OracleGPTModel(cfg, activation_checkpoint_config=none)
    ref32.load_state_dict({k: v.float() for k, v in ref.state_dict().items()})
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, cfg.vocab_size, (batch, seq + 1), generator=g)
    x, y = ids[:, :seq].contiguous(), ids[:, 1:].contiguous()
    loss = ref(x, labels=y).loss
    loss.backward()
    ref32(x, labels=y).loss.backward()
    exact = dict(ref32.named_parameters())
    return float(loss.detach()), [(n, p.grad.detach(), exact[n].grad.detach()) for n, p in ref.named_parameters()]


def _ulp_noise(t: torch.Tensor, seed: int) -> torch.Tensor:
    """t with each element moved by up to one bf16 ulp (a rounding flip)."""
    g = torch.Generator().manual_seed(seed)
    u = torch.rand(t.shape, generator=g) * 2 - 1
    return (t.float() * (1 + u * 2.0 ** -8)).to(t.dtype)


C1_WIDTH = dict(layers=2, hidden_size=256, ffn_hidden_size=688, heads=4, seq_length=128, vocab_size=8192,
                norm_epsilon=1e-5, rope_theta=1e4)
C3 = dict(layers=24, hidden_size=1024, ffn_hidden_size=2736, heads=16, seq_length=512, vocab_size=8192,
          norm_epsilon=1e-5, rope_theta=1e4)


@pytest.mark.parametrize("shape,batch,seq", [(C1_WIDTH, 4, 128), (C3, 1, 512)], ids=["c1_width_2l", "c3_24l"])
def test_bf16_gradient_bar_rejects_planted_mistakes(shape, batch, seq) -> None:
    torch.set_num_threads(min(8, torch.get_num_threads()))
    loss, grads = _oracle_grads(nm.GPTConfig(**shape), batch, seq)
    worst_ref = 0.0
    for i, (name, got, exact) in enumerate(grads):
        ok, _, e_ref = bf16_grad_error(got, got, exact)
        worst_ref = max(worst_ref, e_ref)
        assert ok, name
        assert bf16_grad_error(_ulp_noise(got, i), got, exact)[0], name
        for planted in (torch.zeros_like(got), got * 1.05, got * 0.95):
            assert not bf16_grad_error(planted, got, exact)[0], name
    # the reference's own bf16 error stays below the level at which the bar
    # would stop rejecting a 5% scaling (asserted by assert_bf16_grad too)
    assert worst_ref < BF16_GRAD_MAX_REF_ERR, worst_ref
    # a model with uniform logits (loss ln V) fails the loss bar
    uniform = math.log(shape["vocab_size"])
    with pytest.raises(AssertionError):
        assert_loss_close(uniform, loss, torch.bfloat16)
    assert_loss_close(loss * (1 + 0.5 * loss_rtol(torch.bfloat16)), loss, torch.bfloat16)


@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_scaled_bar_rejects_planted_mistakes_in_small_gradients(reduction) -> None:
    """The LM head + cross entropy in bf16 with reduction "mean": dX is ~1e-5
    and dE ~1e-3, far below the former absolute atol of 1e-2 that a zeroed
    gradient passed.  The scaled bar rejects zeroed and 5%-scaled gradients
    at either reduction and accepts the oracle's with one ulp of noise."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(512, 256, generator=g).bfloat16().requires_grad_(True)
    e = (0.02 * torch.randn(4096, 256, generator=g)).bfloat16().requires_grad_(True)
    t = torch.randint(0, 4096, (512,), generator=g)
    R.cross_entropy_tokens(torch.nn.functional.linear(x, e), t, reduction=reduction).backward()
    for i, grad in enumerate((x.grad, e.grad)):
        if reduction == "mean":
            assert float(grad.float().abs().max()) < 1e-2  # what the former bar could not see
        assert_close_scaled(_ulp_noise(grad, i), grad, torch.bfloat16)
        for planted in (torch.zeros_like(grad), grad * 1.05, grad * 0.95):
            assert not close_scaled(planted, grad, 2e-2, 1e-2)[0]


def test_fp32_bar_rejects_a_relative_error_of_1e_4() -> None:
    g = torch.Generator().manual_seed(2)
    exp = 1e-3 * torch.randn(1000, generator=g)
    assert close_scaled(exp * (1 + 1e-6), exp, 1e-5, 1e-5)[0]
    assert not close_scaled(exp * (1 + 1e-4), exp, 1e-5, 1e-5)[0]
    assert not close_scaled(torch.zeros_like(exp), exp, 1e-5, 1e-5)[0]
