"""GPT model modules on the MI355X kernels, drop-in for models/gpt of the reference.

Class names, constructor arguments, attribute nesting (hence ``state_dict``
keys), initialisation order and forward signatures follow the reference:
``GPTModel`` models/gpt/model.py:40-250, ``GPTLayer`` models/gpt/layer.py:22-137,
``GPTAttention`` models/gpt/attention.py:35-209, ``GPTMLP`` models/gpt/mlp.py:22-78,
``DenseGPTComponents`` models/gpt/factory.py:48-114, the TP=1 layers of
tensor_parallel/layers.py:27-214 and tensor_parallel/embedding.py:22-75.

The model runs on one GPU (tensor, sequence and context parallel size 1; the
reference's collectives are identities there).  ``GPTModel.forward`` runs each
standard layer as one fused block Function:

* ``activation_checkpoint.mode == "full"`` and ``layer_index % block_interval
  == 0`` -> ``CheckpointedBlockFunction`` (saves the block input only, in
  pinned host memory under ``offload_saved_tensors``; recomputes the rest
  inside backward);
* otherwise -> ``EagerBlockFunction`` (same kernels, intermediates kept).

``"selective"`` (training) -> ``SelectiveBlockFunction``: the chosen
sub-blocks checkpointed on their inputs, as the reference's per-sub-block
checkpoints (models/gpt/layer.py:68-89) keep them; a layer the fused block
does not cover runs module by module with those sub-blocks under
non-reentrant ``torch.utils.checkpoint``, as the reference does.  With ``labels`` the loss comes from the chunked
LM-head cross entropy and ``GPTOutput.logits`` is None (full logits are never
built); without labels the logits are returned.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from nano_megatron_amd import functional as Fn
from nano_megatron_amd.block import (
    BlockMeta,
    CheckpointedBlockFunction,
    EagerBlockFunction,
    SelectiveBlockFunction,
    begin_forward_pass,
    pack_adjacent,
)
from nano_megatron_amd.kernels import HipKernelBackend, KernelBackend
from nano_megatron_amd.nn import RotaryEmbedding, activation_checkpoint, activation_rng_context, parallel_dropout

_MISSING = object()


def config_value(config: Any, *names: str, default: Any = _MISSING) -> Any:
    """models/gpt/_config.py:8-17."""
    for name in names:
        if hasattr(config, name):
            return getattr(config, name)
    if default is not _MISSING:
        return default
    raise AttributeError(f"configuration is missing required field (one of: {', '.join(names)})")


def _single_device(parallel: Any, sequence_parallel: bool | None = None) -> None:
    if sequence_parallel:
        raise ValueError("nano_megatron_amd runs on one GPU: sequence parallel is not available")
    if parallel is None:
        return
    for axis in ("tp", "cp", "pp", "ep"):
        group = getattr(parallel, axis, None)
        size = getattr(group, "size", 1) if group is not None else 1
        if size != 1:
            raise ValueError(f"nano_megatron_amd runs on one GPU: {axis} size must be 1, got {size}")


# ---------------------------------------------------------------- TP=1 layers
class ColumnParallelLinear(nn.Module):
    """tensor_parallel/layers.py:27-82 at TP=1: ``self.linear = kernels.linear(...)``."""

    def __init__(self, in_features: int, out_features: int, *, parallel: Any = None,
                 kernels: KernelBackend, bias: bool = True, gather_output: bool = False,
                 sequence_parallel: bool = False, disable_input_gradient_reduce: bool = False,
                 device=None, dtype=None) -> None:
        super().__init__()
        del gather_output, disable_input_gradient_reduce
        _single_device(parallel, sequence_parallel)
        self.in_features = in_features
        self.out_features = out_features
        self.output_size_per_partition = out_features
        self.sequence_parallel = False
        self.linear = kernels.linear(in_features, out_features, bias=bias, device=device, dtype=dtype)

    @property
    def weight(self) -> nn.Parameter:
        return self.linear.weight

    @property
    def bias(self):
        return self.linear.bias

    def forward(self, x: Tensor) -> tuple[Tensor, None]:
        if x.shape[-1] != self.in_features:
            raise ValueError(f"expected input hidden size {self.in_features}, got {x.shape[-1]}")
        return self.linear(x), None


class RowParallelLinear(nn.Module):
    """tensor_parallel/layers.py:85-155 at TP=1."""

    def __init__(self, in_features: int, out_features: int, *, parallel: Any = None,
                 kernels: KernelBackend, bias: bool = True, input_is_parallel: bool = True,
                 sequence_parallel: bool = False, device=None, dtype=None) -> None:
        super().__init__()
        _single_device(parallel, sequence_parallel)
        self.in_features = in_features
        self.out_features = out_features
        self.input_size_per_partition = in_features
        self.input_is_parallel = input_is_parallel
        self.sequence_parallel = False
        self.linear = kernels.linear(in_features, out_features, bias=False, device=device, dtype=dtype)
        self.bias = nn.Parameter(torch.zeros(out_features, device=device, dtype=dtype)) if bias else None

    @property
    def weight(self) -> nn.Parameter:
        return self.linear.weight

    def forward(self, x: Tensor) -> tuple[Tensor, None]:
        if x.shape[-1] != self.in_features:
            raise ValueError(
                f"parallel input must have local hidden size {self.in_features}, got {x.shape[-1]}"
            )
        out = self.linear(x)
        if self.bias is not None:
            out = out + self.bias
        return out, None


class VocabParallelEmbedding(nn.Module):
    """tensor_parallel/embedding.py:22-75 at TP=1 (init N(0, init_std))."""

    def __init__(self, vocab_size: int, hidden_size: int, *, parallel: Any = None,
                 kernels: KernelBackend | None = None, sequence_parallel: bool = False,
                 init_std: float = 0.02, device=None, dtype=None) -> None:
        super().__init__()
        del kernels
        _single_device(parallel, sequence_parallel)
        self.vocab_size = vocab_size
        self.hidden_size = hidden_size
        self.num_embeddings_per_partition = vocab_size
        self.weight = nn.Parameter(torch.empty(vocab_size, hidden_size, device=device, dtype=dtype))
        nn.init.normal_(self.weight, mean=0.0, std=init_std)

    def forward(self, input_ids: Tensor, *, tie: "Fn.TiedGrad | None" = None) -> Tensor:
        return Fn.embedding(self.weight, input_ids, tie)


class VocabParallelLinear(nn.Module):
    """tensor_parallel/layers.py:158-214 at TP=1 (tied weight when given)."""

    def __init__(self, hidden_size: int, vocab_size: int, *, parallel: Any = None,
                 bias: bool = False, sequence_parallel: bool = False,
                 weight: nn.Parameter | None = None, init_std: float = 0.02, device=None,
                 dtype=None) -> None:
        super().__init__()
        _single_device(parallel, sequence_parallel)
        if bias:
            raise ValueError("the fused LM head has no bias (GPTConfig.bias is False)")
        self.hidden_size = hidden_size
        self.vocab_size = vocab_size
        if weight is None:
            self.weight = nn.Parameter(torch.empty(vocab_size, hidden_size, device=device, dtype=dtype))
            nn.init.normal_(self.weight, mean=0.0, std=init_std)
        else:
            if tuple(weight.shape) != (vocab_size, hidden_size):
                raise ValueError(
                    f"tied weight must have shape {(vocab_size, hidden_size)}, got {tuple(weight.shape)}"
                )
            self.weight = weight
        self.bias = None

    def forward(self, x: Tensor) -> Tensor:
        if x.shape[-1] != self.hidden_size:
            raise ValueError(f"expected input hidden size {self.hidden_size}, got {x.shape[-1]}")
        return Fn.linear(x, self.weight)


class VocabParallelCrossEntropy(nn.Module):
    """tensor_parallel/cross_entropy.py:89-123 on logits (used when logits exist)."""

    def __init__(self, *, parallel: Any = None, reduction: str = "none",
                 ignore_index: int = -100, original_vocab_size: int | None = None) -> None:
        super().__init__()
        _single_device(parallel)
        if reduction not in ("none", "mean", "sum"):
            raise ValueError(f"unsupported reduction: {reduction}")
        self.reduction = reduction
        self.ignore_index = ignore_index
        self.original_vocab_size = original_vocab_size

    def forward(self, logits: Tensor, targets: Tensor) -> Tensor:
        """Cross entropy of given logits: the identity matrix as the 'LM head'
        would waste a GEMM, so the logits go through the CE kernels directly."""
        if logits.shape[:-1] != targets.shape:
            raise ValueError(
                "targets must match all non-vocabulary logits dimensions: "
                f"logits={tuple(logits.shape)}, targets={tuple(targets.shape)}"
            )
        vocab = self.original_vocab_size or logits.shape[-1]
        invalid = (targets != self.ignore_index) & ((targets < 0) | (targets >= vocab))
        if torch.any(invalid):
            raise ValueError("targets contain ids outside the original (unpadded) vocabulary")
        loss = _LogitsCrossEntropy.apply(
            logits.reshape(-1, logits.shape[-1]), targets.reshape(-1).long().contiguous(),
            self.ignore_index,
        ).view(targets.shape)
        if self.reduction == "none":
            return loss
        if self.reduction == "sum":
            return loss.sum()
        return loss.sum() / (targets != self.ignore_index).sum().clamp_min(1)


class _LogitsCrossEntropy(torch.autograd.Function):
    """The kernels move 16-byte chunks: a vocabulary that is not a multiple of
    8 runs on a copy padded with -inf columns (zero probability, zero
    gradient)."""

    @staticmethod
    def forward(ctx: Any, logits2: Tensor, targets: Tensor, ignore_index: int) -> Tensor:
        vocab = logits2.shape[1]
        if vocab % 8:
            padded = torch.empty(logits2.shape[0], Fn._round8(vocab), dtype=logits2.dtype, device=logits2.device)
            padded[:, :vocab].copy_(logits2)
            Fn._mask_padding(padded, vocab)
            logits2 = padded
        else:
            logits2 = logits2.contiguous()
        loss = torch.empty(logits2.shape[0], dtype=torch.float32, device=logits2.device)
        lse = torch.empty_like(loss)
        Fn.ce_fwd(logits2, targets, ignore_index, loss, lse)
        ctx.save_for_backward(logits2, targets, lse)
        ctx.ignore_index = ignore_index
        ctx.vocab = vocab
        return loss

    @staticmethod
    def backward(ctx: Any, grad: Tensor):
        logits2, targets, lse = ctx.saved_tensors
        g = logits2.clone()
        Fn.ce_bwd_(g, targets, ctx.ignore_index, lse, grad.float().contiguous())
        return (g if g.shape[1] == ctx.vocab else g[:, : ctx.vocab].contiguous()), None, None


# ---------------------------------------------------------------- attention / MLP
class GPTAttention(nn.Module):
    """MHA/GQA causal self-attention (models/gpt/attention.py:35-209) at TP=CP=1."""

    def __init__(self, config: Any, layer_index: int, *, parallel: Any = None,
                 kernels: KernelBackend, rng: Any = None, cp_attention: Any = None,
                 sequence_parallel: bool | None = None) -> None:
        super().__init__()
        _single_device(parallel, sequence_parallel)
        if cp_attention is not None:
            raise ValueError("context-parallel attention needs several GPUs; use functional.ring_attention")
        self.layer_index = layer_index
        self.kernels = kernels
        self.rng = rng
        self.hidden_size = int(config_value(config, "hidden_size"))
        self.num_heads = int(config_value(config, "heads", "num_attention_heads"))
        self.num_kv_heads = int(config_value(config, "num_kv_heads", "kv_heads", default=self.num_heads))
        if self.hidden_size % self.num_heads:
            raise ValueError("hidden_size must be divisible by the number of attention heads")
        if self.num_heads % self.num_kv_heads:
            raise ValueError("query heads must be divisible by KV heads for grouped-query attention")
        self.head_dim = self.hidden_size // self.num_heads
        self.local_num_heads = self.num_heads
        self.local_num_kv_heads = self.num_kv_heads
        self.kv_hidden_size = self.num_kv_heads * self.head_dim
        self.local_hidden_size = self.hidden_size
        self.dropout = float(config_value(config, "attention_dropout", "dropout", default=0.0))
        bias = bool(config_value(config, "linear_bias", "bias", default=False))
        self.q_proj = ColumnParallelLinear(self.hidden_size, self.hidden_size, kernels=kernels, bias=bias)
        self.k_proj = ColumnParallelLinear(self.hidden_size, self.kv_hidden_size, kernels=kernels, bias=bias)
        self.v_proj = ColumnParallelLinear(self.hidden_size, self.kv_hidden_size, kernels=kernels, bias=bias)
        self.out_proj = RowParallelLinear(self.hidden_size, self.hidden_size, kernels=kernels, bias=bias)
        self.rope = RotaryEmbedding(self.head_dim, theta=float(config_value(config, "rope_theta", default=10_000.0)))

    def forward(self, hidden_states: Tensor, *, position_ids: Tensor | None = None,
                sequence_offset: int = 0, microbatch_index: int = 0) -> Tensor:
        batch, sequence, _ = hidden_states.shape
        q, _ = self.q_proj(hidden_states)
        k, _ = self.k_proj(hidden_states)
        v, _ = self.v_proj(hidden_states)
        q = q.view(batch, sequence, self.num_heads, self.head_dim).transpose(1, 2)
        k = k.view(batch, sequence, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v = v.view(batch, sequence, self.num_kv_heads, self.head_dim).transpose(1, 2)
        tab, positions, offset = _rope_inputs(self.rope, hidden_states.device, sequence,
                                              position_ids, sequence_offset)
        q = Fn.RotaryFunction.apply(Fn._canonical_bhsd(q), tab.cos, tab.sin, positions, offset)
        k = Fn.RotaryFunction.apply(Fn._canonical_bhsd(k), tab.cos, tab.sin, positions, offset)
        with activation_rng_context(
            self.rng if self.training and self.dropout > 0.0 else None, q, layer=self.layer_index,
            microbatch=microbatch_index, global_token_offset=sequence_offset, op="attention.tp=0",
        ):
            context = self.kernels.local_attention(
                q, k, v, causal=True, sequence_offset=sequence_offset,
                dropout_p=self.dropout if self.training else 0.0,
            )
        context = context.transpose(1, 2).contiguous().view(batch, sequence, self.local_hidden_size)
        output, _ = self.out_proj(context)
        return output


@dataclass(frozen=True)
class PositionPlan:
    """RoPE positions of one forward, worked out once for all its layers:
    ``positions`` (int32 [S] or [B, S]) or None for ``offset + arange(S)``, and
    the number of table rows they need; ``first`` is the first position, the
    causal mask's query offset (models/gpt/model.py:199-200)."""

    positions: Tensor | None
    offset: int
    n_pos: int
    first: int


def position_plan(device: torch.device, sequence: int, position_ids: Tensor | None,
                  sequence_offset: int) -> PositionPlan:
    """Default positions arange(offset, offset + S) (models/gpt/model.py:193-198)
    use the offset form (no position tensor), as does a 1-D ``position_ids``
    equal to such a range.  Other ids pass through as an int32 tensor; one host
    read validates and sizes them.  The RoPE tables are indexed by position,
    so a negative position is a ValueError (the reference's rotary embedding
    would accept it, nn/rotary.py:55-70)."""
    if position_ids is None:
        offset = int(sequence_offset)
        if offset < 0:
            raise ValueError(f"sequence_offset must be non-negative, got {offset}")
        return PositionPlan(None, offset, offset + sequence, offset)
    if position_ids.ndim not in (1, 2) or position_ids.shape[-1] != sequence:
        raise ValueError("position_ids sequence length must match the gathered sequence")
    host = position_ids.detach().to("cpu", torch.int64)
    if host.numel() == 0:
        return PositionPlan(None, 0, 1, 0)
    if int(host.min()) < 0:
        raise ValueError("position_ids must be non-negative (the RoPE tables are indexed by position)")
    first = int(host.reshape(-1)[0])
    if host.ndim == 1 and torch.equal(host, torch.arange(first, first + sequence)):
        return PositionPlan(None, first, first + sequence, first)
    pos = position_ids.to(device=device, dtype=torch.int32).contiguous()
    return PositionPlan(pos, 0, int(host.max()) + 1, first)


def _rope_inputs(rope: RotaryEmbedding, device: torch.device, sequence: int,
                 position_ids: Tensor | None, sequence_offset: int):
    """(tables, int32 positions or None, offset) for the RoPE kernel."""
    plan = position_plan(device, sequence, position_ids, sequence_offset)
    return rope.tables(device, plan.n_pos), plan.positions, plan.offset


class GPTMLP(nn.Module):
    """SwiGLU MLP (models/gpt/mlp.py:22-78) at TP=1."""

    def __init__(self, config: Any, layer_index: int, *, parallel: Any = None,
                 kernels: KernelBackend, sequence_parallel: bool | None = None) -> None:
        super().__init__()
        _single_device(parallel, sequence_parallel)
        self.layer_index = layer_index
        hidden = int(config_value(config, "hidden_size"))
        ffn = int(config_value(config, "ffn_hidden_size"))
        bias = bool(config_value(config, "linear_bias", "bias", default=False))
        self.gate_proj = ColumnParallelLinear(hidden, ffn, kernels=kernels, bias=bias)
        self.up_proj = ColumnParallelLinear(hidden, ffn, kernels=kernels, bias=bias)
        self.down_proj = RowParallelLinear(ffn, hidden, kernels=kernels, bias=bias)

    def forward(self, hidden_states: Tensor) -> Tensor:
        gate, _ = self.gate_proj(hidden_states)
        up, _ = self.up_proj(hidden_states)
        output, _ = self.down_proj(Fn.swiglu(gate, up))
        return output


class DenseGPTComponents:
    """models/gpt/factory.py:48-114."""

    def __init__(self, *, cp_attention: Any = None, sequence_parallel: bool | None = None) -> None:
        self.cp_attention = cp_attention
        self.sequence_parallel = sequence_parallel

    def build_attention(self, config, layer_index, *, parallel=None, kernels, rng=None) -> nn.Module:
        return GPTAttention(config, layer_index, parallel=parallel, kernels=kernels, rng=rng,
                            cp_attention=self.cp_attention, sequence_parallel=self.sequence_parallel)

    def build_mlp(self, config, layer_index, *, parallel=None, kernels, parameter_domains=None) -> nn.Module:
        del parameter_domains
        return GPTMLP(config, layer_index, parallel=parallel, kernels=kernels,
                      sequence_parallel=self.sequence_parallel)

    def build_norm(self, config, *, kernels) -> nn.Module:
        return kernels.rms_norm(
            int(config_value(config, "hidden_size")),
            float(config_value(config, "norm_epsilon", "norm_eps", "rms_norm_eps", default=1.0e-6)),
        )


# ---------------------------------------------------------------- layer / model
class GPTLayer(nn.Module):
    """Pre-norm attention + SwiGLU block (models/gpt/layer.py:22-137)."""

    def __init__(self, config: Any, layer_index: int, *, parallel: Any = None,
                 kernels: KernelBackend, cp_attention: Any = None, rng: Any = None,
                 components: Any = None, parameter_domains: Any = None,
                 checkpoint_config: Any = None) -> None:
        super().__init__()
        if components is None:
            components = DenseGPTComponents(cp_attention=cp_attention)
        self.layer_index = layer_index
        self.rng = rng
        self.checkpoint_config = checkpoint_config
        self.input_norm = components.build_norm(config, kernels=kernels)
        self.attention = components.build_attention(config, layer_index, parallel=parallel,
                                                    kernels=kernels, rng=rng)
        self.post_attention_norm = components.build_norm(config, kernels=kernels)
        self.mlp = components.build_mlp(config, layer_index, parallel=parallel, kernels=kernels,
                                        parameter_domains=parameter_domains)
        self.dropout = float(config_value(config, "hidden_dropout", "dropout", default=0.0))

    # -- fused path
    def fusable(self) -> bool:
        return (
            isinstance(self.attention, GPTAttention)
            and isinstance(self.mlp, GPTMLP)
            and type(self.input_norm).__name__ == "RMSNorm"
            and type(self.post_attention_norm).__name__ == "RMSNorm"
            and self.dropout == 0.0
            and self.attention.dropout == 0.0
            # the fused block's bf16 attention kernels take heads of 64 and 128
            and (self.attention.head_dim in (64, 128) or self.input_norm.weight.dtype == torch.float32)
            and all(
                getattr(m, "bias", None) is None
                for m in (self.attention.q_proj.linear, self.attention.k_proj.linear,
                          self.attention.v_proj.linear, self.attention.out_proj,
                          self.mlp.gate_proj.linear, self.mlp.up_proj.linear, self.mlp.down_proj)
            )
        )

    def block_weights(self) -> tuple[Tensor, ...]:
        a, m = self.attention, self.mlp
        return (
            self.input_norm.weight, a.q_proj.weight, a.k_proj.weight, a.v_proj.weight,
            a.out_proj.weight, self.post_attention_norm.weight, m.gate_proj.weight,
            m.up_proj.weight, m.down_proj.weight,
        )

    def block_meta(self, device: torch.device, plan: PositionPlan, sequence_offset: int) -> BlockMeta:
        """The fused block's parameters: ``sequence_offset`` is the causal mask's
        query offset (the reference passes position_ids[0], models/gpt/model.py:
        199-200), ``plan`` the RoPE positions."""
        a = self.attention
        tab = a.rope.tables(device, plan.n_pos)
        return BlockMeta(
            heads=a.num_heads, kv_heads=a.num_kv_heads, head_dim=a.head_dim,
            eps=float(self.input_norm.eps), sequence_offset=int(sequence_offset), cos=tab.cos,
            sin=tab.sin, positions=plan.positions, rope_offset=plan.offset,
        )

    # -- module path (reference semantics, used by selective checkpointing)
    def _selectively_checkpointed(self, name: str) -> bool:
        cfg = self.checkpoint_config
        if cfg is None or getattr(cfg, "mode", "none") != "selective":
            return False
        return name in tuple(getattr(cfg, "selective_ops", ("attention", "mlp")))

    def _run(self, name: str, function, hidden_states: Tensor) -> Tensor:
        if not self._selectively_checkpointed(name) or not self.training:
            return function(hidden_states)
        return activation_checkpoint(
            function, hidden_states, rng=self.rng,
            offload_saved_tensors=bool(getattr(self.checkpoint_config, "offload_saved_tensors", False)),
        )

    def forward(self, hidden_states: Tensor, *, position_ids: Tensor | None = None,
                sequence_offset: int = 0, microbatch_index: int = 0) -> Tensor:
        residual = hidden_states
        normalized = self.input_norm(hidden_states)
        attention_output = self._run(
            "attention",
            lambda x: self.attention(x, position_ids=position_ids, sequence_offset=sequence_offset,
                                     microbatch_index=microbatch_index),
            normalized,
        )
        # residual + dropout (models/gpt/layer.py:114-137) in one pass; the
        # activation offset is the sequence offset (no sequence parallelism)
        hidden_states = parallel_dropout(
            attention_output, self.dropout, training=self.training, rng=self.rng, layer=self.layer_index,
            microbatch=microbatch_index, global_token_offset=sequence_offset, op="attention_residual",
            residual=residual,
        )
        residual = hidden_states
        normalized = self.post_attention_norm(hidden_states)
        return parallel_dropout(
            self._run("mlp", self.mlp, normalized), self.dropout, training=self.training, rng=self.rng,
            layer=self.layer_index, microbatch=microbatch_index, global_token_offset=sequence_offset,
            op="mlp_residual", residual=residual,
        )


@dataclass
class GPTOutput:
    """models/gpt/model.py:31-37."""

    logits: Tensor | None
    loss: Tensor | None
    hidden_states: Tensor


class GPTModel(nn.Module):
    """Decoder-only GPT (models/gpt/model.py:40-250) on one MI355X."""

    def __init__(self, config: Any, *, parallel: Any = None, kernels: KernelBackend | None = None,
                 rng: Any = None, components: Any = None, cp_attention: Any = None,
                 parameter_domains: Any = None, activation_checkpoint_config: Any = None,
                 sequence_parallel: bool | None = None, layer_start: int = 0,
                 layer_end: int | None = None, owns_embedding: bool = True,
                 owns_final_norm: bool = True, owns_lm_head: bool = True,
                 ce_chunk: int = 2048) -> None:
        super().__init__()
        _single_device(parallel, sequence_parallel)
        if cp_attention is not None:
            raise ValueError("context-parallel attention needs several GPUs; use functional.ring_attention")
        kernels = kernels if kernels is not None else HipKernelBackend()
        self.config = config
        self.kernels = kernels
        self.rng = rng
        self.activation_checkpoint_config = activation_checkpoint_config
        self.hidden_size = int(config_value(config, "hidden_size"))
        self.num_layers = int(config_value(config, "layers", "num_layers"))
        self.original_vocab_size = int(config_value(config, "vocab_size"))
        self.padded_vocab_size = self.original_vocab_size
        self.dropout = float(config_value(config, "embedding_dropout", "dropout", default=0.0))
        self.ce_chunk = int(ce_chunk)
        self.layer_start = layer_start
        self.layer_end = self.num_layers if layer_end is None else layer_end
        if not 0 <= self.layer_start <= self.layer_end <= self.num_layers:
            raise ValueError(
                f"invalid layer range [{self.layer_start}, {self.layer_end}) for {self.num_layers} layers"
            )
        if self.layer_start == self.layer_end:
            raise ValueError("a GPT stage must own at least one transformer layer")
        init_std = float(config_value(config, "init_std", default=0.02))
        self.embedding = (
            VocabParallelEmbedding(self.padded_vocab_size, self.hidden_size, kernels=kernels,
                                   init_std=init_std)
            if owns_embedding else None
        )
        if components is None:
            components = DenseGPTComponents()
        self.layers = nn.ModuleList([
            GPTLayer(config, i, parallel=parallel, kernels=kernels, rng=rng, components=components,
                     parameter_domains=parameter_domains, checkpoint_config=activation_checkpoint_config)
            for i in range(self.layer_start, self.layer_end)
        ])
        self.final_norm = components.build_norm(config, kernels=kernels) if owns_final_norm else None
        tied = None
        if bool(config_value(config, "tie_embeddings", default=True)) and self.embedding is not None:
            tied = self.embedding.weight
        self.lm_head = (
            VocabParallelLinear(self.hidden_size, self.padded_vocab_size, weight=tied, init_std=init_std)
            if owns_lm_head else None
        )
        self.loss_fn = (
            VocabParallelCrossEntropy(reduction="mean", original_vocab_size=self.original_vocab_size)
            if owns_lm_head else None
        )

    def _pack_block_weights(self) -> None:
        """Keep each layer's [Wq; Wk; Wv] and [Wg; Wu] adjacent in memory so the
        fused projections read them in place (a no-op once packed)."""
        for layer in self.layers:
            if layer.fusable():
                a, m = layer.attention, layer.mlp
                pack_adjacent((a.q_proj.weight, a.k_proj.weight, a.v_proj.weight))
                pack_adjacent((m.gate_proj.weight, m.up_proj.weight))

    def _checkpoint_layer(self, layer: GPTLayer) -> bool:
        """models/gpt/model.py:162-170."""
        config = self.activation_checkpoint_config
        if config is None or getattr(config, "mode", "none") != "full" or not self.training:
            return False
        interval = int(getattr(config, "block_interval", 1))
        if interval <= 0:
            raise ValueError("activation checkpoint block_interval must be positive")
        return layer.layer_index % interval == 0

    def forward(self, input_ids: Tensor | None = None, *, labels: Tensor | None = None,
                position_ids: Tensor | None = None, hidden_states: Tensor | None = None,
                microbatch_index: int = 0) -> GPTOutput:
        # the loss's target-range check, enqueued before the layers (see TargetCheck);
        # a host wait cannot be captured in a HIP graph, so under capture the
        # caller validates the targets before each replay (CapturedTrainStep)
        check = None
        if labels is not None and self.lm_head is not None:
            if labels.is_cuda and torch.cuda.is_current_stream_capturing():
                check = False
            else:
                check = Fn.TargetCheck(labels, self.lm_head.weight.shape[0], Fn.IGNORE_INDEX)
        if self.embedding is not None:
            Fn.require_precision(self.embedding.weight)
        # the tied LM head passes its table gradient to the embedding's backward
        tie = None
        if (labels is not None and self.embedding is not None and self.lm_head is not None
                and self.lm_head.weight is self.embedding.weight and torch.is_grad_enabled()):
            tie = Fn.TiedGrad()
        if self.embedding is not None:
            if input_ids is None:
                raise ValueError("the first pipeline stage requires input_ids")
            hidden_states = self.embedding(input_ids, tie=tie)
        elif hidden_states is None:
            raise ValueError("a non-first pipeline stage requires hidden_states")
        Fn._require_gpu(hidden_states)
        Fn.require_precision(hidden_states)
        sequence = hidden_states.shape[1]
        # positions and the causal offset once per forward (models/gpt/model.py:193-200)
        plan = position_plan(hidden_states.device, sequence, position_ids, 0)
        offset = plan.first
        if plan.positions is None:
            position_ids = None  # the offset form: the module path builds the same range

        if self.embedding is not None:
            # models/gpt/model.py:203-212 (no sequence parallelism: the offset is the position)
            hidden_states = parallel_dropout(
                hidden_states, self.dropout, training=self.training, rng=self.rng, layer=0,
                microbatch=microbatch_index, global_token_offset=offset, op="embedding",
            )

        self._pack_block_weights()
        begin_forward_pass(hidden_states.device)
        mode = getattr(self.activation_checkpoint_config, "mode", "none")
        offload = bool(getattr(self.activation_checkpoint_config, "offload_saved_tensors", False))
        for layer in self.layers:
            if layer.fusable():
                weights = layer.block_weights()
                if any(w.dtype != hidden_states.dtype for w in weights):
                    raise ValueError(
                        "the fused block computes in the parameter dtype: parameters "
                        f"{weights[1].dtype} vs activations {hidden_states.dtype}"
                    )
                meta = layer.block_meta(hidden_states.device, plan, offset)
                if mode == "selective" and self.training:
                    ops = tuple(getattr(self.activation_checkpoint_config, "selective_ops", ("attention", "mlp")))
                    hidden_states = SelectiveBlockFunction.apply(hidden_states, meta, ops, offload, *weights)
                elif self._checkpoint_layer(layer):
                    hidden_states = CheckpointedBlockFunction.apply(hidden_states, meta, offload, *weights)
                else:
                    hidden_states = EagerBlockFunction.apply(hidden_states, meta, *weights)
            elif self._checkpoint_layer(layer):
                # a layer the fused block does not cover (dropout, biases, other
                # components): torch's checkpoint of the module path
                # (models/gpt/model.py:217-235)
                hidden_states = activation_checkpoint(
                    lambda x, current=layer: current(x, position_ids=position_ids, sequence_offset=offset,
                                                     microbatch_index=microbatch_index),
                    hidden_states, rng=self.rng, offload_saved_tensors=offload,
                )
            else:
                hidden_states = layer(hidden_states, position_ids=position_ids,
                                      sequence_offset=offset, microbatch_index=microbatch_index)

        if self.final_norm is not None:
            hidden_states = self.final_norm(hidden_states)
        logits = loss = None
        if labels is not None:
            if self.lm_head is None:
                raise ValueError("labels may only be supplied to a stage that owns the LM head")
            loss = Fn.lm_head_cross_entropy(hidden_states, self.lm_head.weight, labels,
                                            reduction="mean", chunk=self.ce_chunk, tie=tie,
                                            validate=check)
        elif self.lm_head is not None:
            logits = self.lm_head(hidden_states)
        return GPTOutput(logits=logits, loss=loss, hidden_states=hidden_states)
