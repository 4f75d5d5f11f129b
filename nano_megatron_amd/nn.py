"""RMSNorm, RoPE and the activation-checkpoint helper, backed by libnmb.so.

Mirrors nn/norms.py:13-44, nn/rotary.py:9-73 and
nn/activation_checkpoint.py:73-131 of the reference: same constructor
arguments, validation messages and outputs.
"""

from __future__ import annotations

from collections.abc import Callable
from contextlib import nullcontext
from typing import Any, TypeVar

import torch
from torch import Tensor, nn
from torch.utils.checkpoint import checkpoint as torch_checkpoint

from nano_megatron_amd import functional as Fn

T = TypeVar("T")


class RMSNorm(nn.Module):
    """Root-mean-square normalization with a learned per-channel scale (nn/norms.py:13-44)."""

    def __init__(
        self,
        hidden_size: int,
        eps: float = 1.0e-6,
        *,
        device: torch.device | str | None = None,
        dtype: torch.dtype | None = None,
    ) -> None:
        super().__init__()
        if hidden_size <= 0:
            raise ValueError(f"hidden_size must be positive, got {hidden_size}")
        if eps <= 0:
            raise ValueError(f"eps must be positive, got {eps}")
        self.hidden_size = hidden_size
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))

    def forward(self, x: Tensor) -> Tensor:
        if x.shape[-1] != self.hidden_size:
            raise ValueError(
                f"expected the last dimension to be {self.hidden_size}, got {x.shape[-1]}"
            )
        return Fn.rms_norm(x, self.weight, self.eps)

    def extra_repr(self) -> str:
        return f"hidden_size={self.hidden_size}, eps={self.eps}"


class RotaryEmbedding(nn.Module):
    """cos/sin values for explicit position ids (nn/rotary.py:41-73).

    The tables come from ``nmb_rope_table`` (cos/sin of ``p * inv_freq`` in
    fp32, inv_freq computed as nn/rotary.py:52 does) and are returned in the
    reference's ``cat(f, f)`` layout cast to ``dtype``.
    """

    def __init__(self, dim: int, theta: float = 10_000.0) -> None:
        super().__init__()
        if dim <= 0 or dim % 2:
            raise ValueError(f"RoPE dim must be a positive even integer, got {dim}")
        if theta <= 0:
            raise ValueError(f"theta must be positive, got {theta}")
        self.dim = dim
        self.theta = theta

    def tables(self, device: torch.device, n_pos: int) -> Fn.RopeTables:
        return Fn.RopeTables.get(device, self.dim, self.theta, n_pos)

    def forward(
        self,
        position_ids: Tensor,
        *,
        device: torch.device | None = None,
        dtype: torch.dtype | None = None,
    ) -> tuple[Tensor, Tensor]:
        if position_ids.ndim not in (1, 2):
            raise ValueError("position_ids must have shape [sequence] or [batch, sequence]")
        target = device if device is not None else position_ids.device
        pos = position_ids.to(device=target, dtype=torch.long)
        n_pos = int(pos.max().item()) + 1 if pos.numel() else 1
        tab = self.tables(torch.device(target), n_pos)
        half_cos = tab.cos[pos]
        half_sin = tab.sin[pos]
        out_dtype = dtype if dtype is not None else torch.get_default_dtype()
        cos = torch.cat((half_cos, half_cos), dim=-1).to(out_dtype)
        sin = torch.cat((half_sin, half_sin), dim=-1).to(out_dtype)
        return cos, sin

    def extra_repr(self) -> str:
        return f"dim={self.dim}, theta={self.theta}"


def apply_rotary_pos_emb(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    """RoPE for [B,H,S,D] q and k (nn/rotary.py:27-38).

    cos/sin are the reference-layout tables ([S,D] or [B,S,D], ``emb = cat(f, f)``);
    only their first half is read.
    """
    if q.ndim != 4 or k.ndim != 4:
        raise ValueError("q and k must use [batch, heads, sequence, head_dim] layout")
    if q.shape[-1] != k.shape[-1]:
        raise ValueError("q and k must have the same head_dim")
    if q.shape[-1] % 2:
        raise ValueError("RoPE head_dim must be even")
    ct, st, pos = Fn.rope_tables_from_cos_sin(cos, sin, q.shape[0], q.shape[2])
    q = Fn._canonical_bhsd(q)
    k = Fn._canonical_bhsd(k)
    return (
        Fn.RotaryFunction.apply(q, ct, st, pos, 0),
        Fn.RotaryFunction.apply(k, ct, st, pos, 0),
    )


def _offload_context(*, pin_memory: bool, non_blocking: bool):
    """Saved-tensor CPU offload (nn/activation_checkpoint.py:24-41)."""

    def pack(tensor: Tensor):
        if tensor.device.type == "cpu":
            return tensor
        cpu = torch.empty(tensor.shape, dtype=tensor.dtype, pin_memory=pin_memory)
        cpu.copy_(tensor.detach(), non_blocking=non_blocking)
        return (cpu, tensor.device)

    def unpack(value):
        if isinstance(value, Tensor):
            return value
        cpu, device = value
        return cpu.to(device, non_blocking=non_blocking)

    return torch.autograd.graph.saved_tensors_hooks(pack, unpack)


def activation_checkpoint(
    function: Callable[..., T],
    *args: Any,
    rng: Any | None = None,
    offload_saved_tensors: bool = False,
    pin_memory: bool = True,
    non_blocking: bool = True,
    **kwargs: Any,
) -> T:
    """Non-reentrant checkpoint of an arbitrary function (nn/activation_checkpoint.py:73-100).

    Used for the selective mode; the full mode of GPTModel uses the fused
    CheckpointedBlockFunction instead.  ``rng`` is accepted for signature
    compatibility: the hot path has no random ops at dropout 0.
    """
    del rng
    context = (
        _offload_context(pin_memory=pin_memory, non_blocking=non_blocking)
        if offload_saved_tensors
        else nullcontext()
    )
    with context:
        return torch_checkpoint(
            lambda *inputs: function(*inputs, **kwargs), *args, use_reentrant=False,
            preserve_rng_state=True,
        )
