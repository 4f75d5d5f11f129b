"""RMSNorm, RoPE, dropout and the activation-checkpoint helper, backed by libnmb.so.

Mirrors nn/norms.py:13-44, nn/rotary.py:9-73, nn/dropout.py:14-70 and
nn/activation_checkpoint.py:44-131 of the reference: same constructor
arguments, validation messages and outputs.
"""

from __future__ import annotations

import copy
from collections.abc import Callable, Iterator
from contextlib import contextmanager, nullcontext
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


def _rng_replaying(function: Callable[..., T], rng: Any | None) -> Callable[..., T]:
    """nn/activation_checkpoint.py:44-70: a stateful RNG tracker (anything with
    state_dict / load_state_dict) starts the first forward and the recompute
    from the same state, and is left where the first forward left it.  torch's
    own CPU generator, which the dropout seeds come from, is replayed by
    torch's checkpoint itself (preserve_rng_state)."""
    if rng is None or not hasattr(rng, "state_dict") or not hasattr(rng, "load_state_dict"):
        return function
    start = copy.deepcopy(rng.state_dict())
    after_first: list[Any] = []

    def replaying(*args: Any, **kwargs: Any) -> T:
        rng.load_state_dict(copy.deepcopy(start))
        try:
            return function(*args, **kwargs)
        finally:
            if after_first:
                rng.load_state_dict(copy.deepcopy(after_first[0]))
            else:
                after_first.append(copy.deepcopy(rng.state_dict()))

    return replaying


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

    Used for the selective mode and for layers the fused block does not cover
    (dropout, biases); the full mode of fusable layers uses the fused
    CheckpointedBlockFunction instead.  ``rng``: a stateful tracker replayed
    across the recompute.
    """
    function = _rng_replaying(function, rng)
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


class ActivationCheckpoint(nn.Module):
    """nn/activation_checkpoint.py:103-131: a module whose forward runs the
    wrapped module under activation_checkpoint with the stored options."""

    def __init__(self, module: nn.Module, *, rng: Any | None = None, offload_saved_tensors: bool = False,
                 pin_memory: bool = True, non_blocking: bool = True) -> None:
        super().__init__()
        self.module = module
        self.rng = rng
        self.offload_saved_tensors = offload_saved_tensors
        self.pin_memory = pin_memory
        self.non_blocking = non_blocking

    def forward(self, *args: Any, **kwargs: Any) -> Any:
        return activation_checkpoint(self.module, *args, rng=self.rng,
                                     offload_saved_tensors=self.offload_saved_tensors,
                                     pin_memory=self.pin_memory, non_blocking=self.non_blocking, **kwargs)


@contextmanager
def activation_rng_context(rng: Any | None, tensor: Tensor, *, layer: int, microbatch: int,
                           global_token_offset: int, op: str) -> Iterator[None]:
    """nn/dropout.py:14-44: run one logical random operation inside the stream
    ``rng.fork`` derives from (layer, microbatch, global_token_offset, op), so
    its dropout mask does not depend on what ran before it.  The kernels draw
    their mask keys from torch's default CPU generator (functional.dropout_seed),
    the generator the fork reseeds; no CUDA generator is involved, so none is
    forked.  Without an rng (or one without ``fork``) the default CPU
    generator's running stream is used and advanced; the reference's F.dropout
    then advances the CUDA generator instead, so later CPU randomness differs
    from a reference run with the same seed."""
    del tensor
    if rng is None or not hasattr(rng, "fork"):
        yield
        return
    with rng.fork("activation", components=(layer, microbatch, global_token_offset, op), cuda_devices=(),
                  advance=False):
        yield


def parallel_dropout(tensor: Tensor, p: float, *, training: bool, rng: Any | None, layer: int,
                     microbatch: int, global_token_offset: int, op: str,
                     residual: Tensor | None = None) -> Tensor:
    """nn/dropout.py:47-70 (``F.dropout`` in training mode under the forked
    stream), plus the residual add that follows it in GPTLayer.forward
    (models/gpt/layer.py:114-137) fused into the same pass when ``residual``
    is given.  Identity (or the plain add) when not training or at p = 0."""
    if not training or p == 0.0:
        return tensor if residual is None else residual + tensor
    with activation_rng_context(rng, tensor, layer=layer, microbatch=microbatch,
                                global_token_offset=global_token_offset, op=op):
        return Fn.dropout_add(tensor, p, residual=residual)
