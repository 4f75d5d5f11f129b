"""PyTorch-CPU restatement of the reference hot path (test infrastructure only).

Citations are ``file:line`` under the reference's ``src/nano_megatron/``.
The modules keep the reference's parameter nesting so that their
``state_dict`` keys equal the reference's (``layers.{i}.attention.q_proj.
linear.weight``, ``layers.{i}.mlp.gate_proj.linear.weight``,
``layers.{i}.input_norm.weight``, ``embedding.weight``, ...), which lets a test
load one set of weights into this oracle and into ``nano_megatron_amd``.

Tensor parallel, sequence parallel and context parallel all run at size 1 here,
where every collective on the path is an identity
(tensor_parallel/sequence_parallel.py:37-39, 46-48, 55-57).  Dropout is the
identity at p = 0 (nn/dropout.py:60-61), which is the only value the configs
use; for p > 0 the reference draws its masks from torch's Philox stream,
which no other generator reproduces, so the functions below take the keep
mask of the library's SplitMix64 stream (``dropout_keep``) and apply it with
the reference's arithmetic.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Sequence

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor, nn
from torch.utils.checkpoint import checkpoint as torch_checkpoint


def _cfg(config: Any, *names: str, default: Any = None) -> Any:
    """Duck-typed config lookup in the manner of models/gpt/_config.py:8-17."""
    for name in names:
        if hasattr(config, name):
            value = getattr(config, name)
            if value is not None:
                return value
    return default


# ---------------------------------------------------------------- RMSNorm
def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """RMSNorm forward with the reference's cast placement (nn/norms.py:38-41).

    Statistics in fp32; the normalised value is rounded to the input dtype
    before the multiply by the (input-dtype) weight.
    """
    input_dtype = x.dtype
    variance = x.float().square().mean(dim=-1, keepdim=True)
    normalized = x.float() * torch.rsqrt(variance + eps)
    return normalized.to(input_dtype) * weight.to(input_dtype)


class OracleRMSNorm(nn.Module):
    """nn/norms.py:13-44 (weight initialised to ones, shape [hidden])."""

    def __init__(self, hidden_size: int, eps: float, dtype: torch.dtype | None = None) -> None:
        super().__init__()
        if hidden_size <= 0:
            raise ValueError(f"hidden_size must be positive, got {hidden_size}")
        if eps <= 0:
            raise ValueError(f"eps must be positive, got {eps}")
        self.hidden_size = hidden_size
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size, dtype=dtype))

    def forward(self, x: Tensor) -> Tensor:
        if x.shape[-1] != self.hidden_size:
            raise ValueError(
                f"expected the last dimension to be {self.hidden_size}, got {x.shape[-1]}"
            )
        return rms_norm(x, self.weight, self.eps)


# ---------------------------------------------------------------- RoPE
def rope_inv_freq(dim: int, theta: float) -> Tensor:
    """``1 / theta ** (arange(0, dim, 2) / dim)`` in fp32 (nn/rotary.py:52)."""
    return 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))


def rope_cos_sin(
    position_ids: Tensor, dim: int, theta: float, dtype: torch.dtype
) -> tuple[Tensor, Tensor]:
    """cos/sin tables [S, D] (or [B, S, D]) cast to ``dtype`` (nn/rotary.py:55-70).

    ``emb = cat(f, f)``: NeoX-style halves, not interleaved pairs.
    """
    if position_ids.ndim not in (1, 2):
        raise ValueError("position_ids must have shape [sequence] or [batch, sequence]")
    positions = position_ids.to(dtype=torch.float32)
    frequencies = positions.unsqueeze(-1) * rope_inv_freq(dim, theta)
    embeddings = torch.cat((frequencies, frequencies), dim=-1)
    return embeddings.cos().to(dtype), embeddings.sin().to(dtype)


def _rotate_half(x: Tensor) -> Tensor:
    """``cat(-x2, x1)`` over the two halves of the last dim (nn/rotary.py:9-11)."""
    first, second = x.chunk(2, dim=-1)
    return torch.cat((-second, first), dim=-1)


def apply_rotary_pos_emb(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    """``q*cos + rot(q)*sin`` for [B,H,S,D] tensors (nn/rotary.py:27-38).

    In bf16 this rounds after each multiply and after the add, as the reference's
    three separate tensor ops do.
    """
    if q.ndim != 4 or k.ndim != 4:
        raise ValueError("q and k must use [batch, heads, sequence, head_dim] layout")
    if q.shape[-1] != k.shape[-1]:
        raise ValueError("q and k must have the same head_dim")
    if q.shape[-1] % 2:
        raise ValueError("RoPE head_dim must be even")

    def shape(t: Tensor) -> Tensor:
        if t.ndim == 2:
            return t.unsqueeze(0).unsqueeze(0)
        if t.ndim == 3:
            return t.unsqueeze(1)
        raise ValueError("RoPE cos/sin tensors must be [S,D] or [B,S,D]")

    cos = shape(cos).to(dtype=q.dtype)
    sin = shape(sin).to(dtype=q.dtype)
    return (q * cos) + (_rotate_half(q) * sin), (k * cos) + (_rotate_half(k) * sin)


class OracleRotaryEmbedding(nn.Module):
    """nn/rotary.py:41-73."""

    def __init__(self, dim: int, theta: float = 10_000.0) -> None:
        super().__init__()
        if dim <= 0 or dim % 2:
            raise ValueError(f"RoPE dim must be a positive even integer, got {dim}")
        self.dim = dim
        self.theta = theta

    def forward(self, position_ids: Tensor, *, dtype: torch.dtype) -> tuple[Tensor, Tensor]:
        return rope_cos_sin(position_ids, self.dim, self.theta, dtype)


# ---------------------------------------------------------------- attention
def local_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    *,
    causal: bool = True,
    sequence_offset: int = 0,
    scale: float | None = None,
    attention_mask: Tensor | None = None,
    dropout_p: float = 0.0,
    dropout_seed: int = 0,
) -> Tensor:
    """``TorchKernelBackend.local_attention`` (nn/kernels/torch_backend.py:25-76).

    GQA by ``repeat_interleave`` of K/V heads (:51-58); causal by ``is_causal``
    when there is no mask and the offset is 0, else by an explicit
    ``key_pos <= offset + query_pos`` mask, ANDed with ``attention_mask`` when
    one is given (:60-66); then SDPA with that mask (:68-76): a boolean mask
    keeps the True entries, a floating mask is added to the scores.  With
    ``dropout_p`` > 0 (:73), torch's math SDPA applies the keep mask
    ``dropout_keep(dropout_seed, [B, Hq, Sq, Sk], dropout_p)`` to the
    normalised probabilities and scales by 1 / (1 - p).
    """
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k and v must have [batch, heads, sequence, head_dim] shape")
    if k.shape != v.shape:
        raise ValueError("k and v must have identical shapes")
    if q.shape[0] != k.shape[0] or q.shape[-1] != k.shape[-1]:
        raise ValueError("q and k/v must agree on batch size and head_dim")
    if q.shape[1] != k.shape[1]:
        if q.shape[1] % k.shape[1]:
            raise ValueError(
                f"query heads ({q.shape[1]}) must be divisible by KV heads ({k.shape[1]})"
            )
        repeat = q.shape[1] // k.shape[1]
        k = k.repeat_interleave(repeat, dim=1)
        v = v.repeat_interleave(repeat, dim=1)
    is_causal = causal and attention_mask is None and sequence_offset == 0
    mask = attention_mask
    if causal and not is_causal:
        query_positions = sequence_offset + torch.arange(q.shape[-2])
        key_positions = torch.arange(k.shape[-2])
        causal_mask = key_positions.unsqueeze(0) <= query_positions.unsqueeze(1)
        mask = causal_mask if mask is None else (mask & causal_mask)
    if dropout_p:
        keep = dropout_keep(dropout_seed, (q.shape[0], q.shape[1], q.shape[2], k.shape[2]), dropout_p)
        if mask is not None and mask.dtype == torch.bool:
            # the math kernel takes additive masks: SDPA's own conversion (False -> -inf)
            mask = torch.zeros(mask.shape, dtype=q.dtype).masked_fill(~mask, float("-inf"))
        out, _ = torch.ops.aten._scaled_dot_product_attention_math(
            q, k, v, mask, float(np.float32(dropout_p)), is_causal, keep, scale=scale)
        return out
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=is_causal, scale=scale)


# ---------------------------------------------------------------- dropout masks
_SM_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_SM_MUL1 = np.uint64(0xBF58476D1CE4E5B9)
_SM_MUL2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, counters: np.ndarray) -> np.ndarray:
    """Output ``counter + 1`` of SplitMix64 seeded with ``seed`` (Steele, Lea
    and Flood, OOPSLA 2014; the mixing of Vigna's splitmix64.c), for each
    counter: z = seed + (counter + 1) * 0x9E3779B97F4A7C15, two
    xor-shift-multiply rounds (30, 27) and a final xor-shift (31), mod 2^64."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.asarray(counters, dtype=np.uint64) + np.uint64(1)) * _SM_GAMMA
        z = (z ^ (z >> np.uint64(30))) * _SM_MUL1
        z = (z ^ (z >> np.uint64(27))) * _SM_MUL2
        return z ^ (z >> np.uint64(31))


def dropout_bits(seed: int, n: int) -> np.ndarray:
    """The 32-bit draw of elements 0..n-1: the low (even index) or high (odd
    index) half of splitmix64(seed, index >> 1)."""
    idx = np.arange(n, dtype=np.uint64)
    z = splitmix64(seed, idx >> np.uint64(1))
    return np.where((idx & np.uint64(1)) == 1, z >> np.uint64(32), z & np.uint64(0xFFFFFFFF)).astype(np.uint32)


def dropout_keep(seed: int, shape: Sequence[int], p: float) -> Tensor:
    """Boolean keep mask over ``shape`` (row-major element index): kept iff
    the draw is >= floor(p * 2^32), p taken in float32 as the kernels take it."""
    threshold = int(float(np.float32(p)) * 4294967296.0)
    n = int(np.prod(shape)) if len(shape) else 1
    return torch.from_numpy(dropout_bits(seed, n) >= threshold).reshape(tuple(shape))


def dropout_scale(p: float) -> float:
    """1 / (1 - p) rounded to float32, the kept elements' factor."""
    return float(np.float32(1.0 / (1.0 - float(np.float32(p)))))


def dropout_add(x: Tensor, p: float, seed: int, residual: Tensor | None = None) -> Tensor:
    """``residual + F.dropout(x, p)`` with the keep mask of ``seed``
    (nn/dropout.py:47-70; models/gpt/layer.py:114-137)."""
    return dropout_apply(x, dropout_keep(seed, x.shape, p), p, residual)


def dropout_apply(x: Tensor, keep: Tensor, p: float, residual: Tensor | None = None) -> Tensor:
    """F.dropout's arithmetic on the GPU for a given keep mask: x * (1 / (1 - p))
    in float32, rounded to x's dtype (0 where dropped); then ``residual +`` that,
    rounded once more."""
    keep = keep.to(x.device)
    scaled = x.float() * torch.tensor(dropout_scale(p), dtype=torch.float32, device=x.device)
    y = torch.where(keep, scaled, torch.zeros((), dtype=torch.float32, device=x.device)).to(x.dtype)
    if residual is None:
        return y
    return (residual.float() + y.float()).to(x.dtype)


def _ring_block_mask(sq: int, sk: int, query_offset: int, key_offset: int) -> Tensor:
    """Absolute-position causal mask ``key <= query`` (context_parallel/ring.py:58-79)."""
    qpos = torch.arange(query_offset, query_offset + sq)
    kpos = torch.arange(key_offset, key_offset + sk)
    return (kpos.unsqueeze(0) <= qpos.unsqueeze(1)).view(1, 1, sq, sk)


def _expand_kv(t: Tensor, heads: int) -> Tensor:
    """context_parallel/ring.py:40-48."""
    repeat = heads // t.size(1)
    return t if repeat == 1 else t.repeat_interleave(repeat, dim=1)


def _collapse_kv(g: Tensor, kv_heads: int) -> Tensor:
    """context_parallel/ring.py:51-55."""
    b, h, s, d = g.shape
    repeat = h // kv_heads
    return g if repeat == 1 else g.reshape(b, kv_heads, repeat, s, d).sum(dim=2)


def ring_attention_forward(
    q: Tensor,
    kv_blocks: Sequence[tuple[Tensor, Tensor]],
    key_offsets: Sequence[int],
    *,
    causal: bool,
    query_offset: int,
) -> tuple[Tensor, Tensor]:
    """One ring rank's forward, blocks visited in ring order (context_parallel/ring.py:104-166).

    Computes in fp32 (fp64 for fp64 inputs, :18-19); per block: scores, the
    absolute-position mask, then the online max/sum merge with ``nan_to_num``
    for fully-masked rows (:145-158).  Returns ``(output in q.dtype, lse)``
    with lse shaped [B, H, Sq, 1].
    """
    cdt = torch.float64 if q.dtype == torch.float64 else torch.float32
    qc = q.to(cdt)
    running_max = torch.full((*q.shape[:-1], 1), -torch.inf, dtype=cdt)
    running_sum = torch.zeros_like(running_max)
    acc = torch.zeros_like(qc)
    scale = 1.0 / math.sqrt(q.size(-1))
    for (kb, vb), koff in zip(kv_blocks, key_offsets):
        ke = _expand_kv(kb, q.size(1)).to(cdt)
        ve = _expand_kv(vb, q.size(1)).to(cdt)
        scores = torch.matmul(qc, ke.transpose(-1, -2)).mul_(scale)
        if causal:
            valid = _ring_block_mask(q.size(-2), kb.size(-2), query_offset, koff)
            scores.masked_fill_(~valid, -torch.inf)
        block_max = scores.amax(dim=-1, keepdim=True)
        new_max = torch.maximum(running_max, block_max)
        old_scale = torch.where(
            torch.isfinite(running_max), torch.exp(running_max - new_max), torch.zeros_like(running_max)
        )
        p = torch.nan_to_num(torch.exp(scores - new_max), nan=0.0)
        acc.mul_(old_scale).add_(torch.matmul(p, ve))
        running_sum.mul_(old_scale).add_(p.sum(dim=-1, keepdim=True))
        running_max = new_max
    tiny = torch.finfo(cdt).tiny
    out = acc / running_sum.clamp_min(tiny)
    lse = running_max + torch.log(running_sum.clamp_min(tiny))
    return out.to(q.dtype), lse


def ring_attention_backward(
    grad_output: Tensor,
    q: Tensor,
    kv_blocks: Sequence[tuple[Tensor, Tensor]],
    key_offsets: Sequence[int],
    output: Tensor,
    lse: Tensor,
    *,
    causal: bool,
    query_offset: int,
) -> tuple[Tensor, list[Tensor], list[Tensor]]:
    """One ring rank's backward (context_parallel/ring.py:169-250).

    ``delta = rowsum(dO*O)``; per block ``P = exp(S - lse)``,
    ``dS = P (dP - delta)``; dQ accumulates locally, dK/dV per block.
    """
    cdt = torch.float64 if q.dtype == torch.float64 else torch.float32
    qc, go, oc = q.to(cdt), grad_output.to(cdt), output.to(cdt)
    delta = (go * oc).sum(dim=-1, keepdim=True)
    dq = torch.zeros_like(qc)
    scale = 1.0 / math.sqrt(q.size(-1))
    dks, dvs = [], []
    for (kb, vb), koff in zip(kv_blocks, key_offsets):
        kv_heads = kb.size(1)
        ke = _expand_kv(kb.to(cdt), q.size(1))
        ve = _expand_kv(vb.to(cdt), q.size(1))
        scores = torch.matmul(qc, ke.transpose(-1, -2)).mul_(scale)
        if causal:
            valid = _ring_block_mask(q.size(-2), kb.size(-2), query_offset, koff)
            scores.masked_fill_(~valid, -torch.inf)
        p = torch.nan_to_num(torch.exp(scores - lse.to(cdt)), nan=0.0)
        dp = torch.matmul(go, ve.transpose(-1, -2))
        ds = p * (dp - delta)
        dq.add_(torch.matmul(ds, ke).mul_(scale))
        dks.append(_collapse_kv(torch.matmul(ds.transpose(-1, -2), qc).mul_(scale), kv_heads).to(kb.dtype))
        dvs.append(_collapse_kv(torch.matmul(p.transpose(-1, -2), go), kv_heads).to(vb.dtype))
    return dq.to(q.dtype), dks, dvs


# ---------------------------------------------------------------- MLP
def swiglu(gate: Tensor, up: Tensor) -> Tensor:
    """``silu(gate) * up`` (models/gpt/mlp.py:77)."""
    return F.silu(gate) * up


# ---------------------------------------------------------------- cross entropy
class _TokenCrossEntropy(torch.autograd.Function):
    """``_VocabParallelCrossEntropy`` at TP=1 (tensor_parallel/cross_entropy.py:30-86).

    fp32 softmax for bf16/fp16 logits (:48-52); loss = log(sum exp(shifted)) -
    shifted[target], zero for ignored targets (:57-66); the gradient is
    ``(softmax - onehot) * g`` cast back to the logits dtype (:74-86).
    """

    @staticmethod
    def forward(ctx: Any, logits: Tensor, targets: Tensor, ignore_index: int) -> Tensor:
        z = logits.float() if logits.dtype in (torch.float16, torch.bfloat16) else logits
        zmax = z.max(dim=-1).values
        shifted = z - zmax.unsqueeze(-1)
        ignored = targets == ignore_index
        outside = (targets < 0) | (targets >= z.shape[-1]) | ignored
        local_t = targets.masked_fill(outside, 0)
        predicted = shifted.gather(-1, local_t.unsqueeze(-1)).squeeze(-1).masked_fill(outside, 0.0)
        exp = shifted.exp()
        sum_exp = exp.sum(dim=-1)
        softmax = exp / sum_exp.unsqueeze(-1)
        loss = (sum_exp.log() - predicted).masked_fill(ignored, 0.0)
        ctx.save_for_backward(softmax, local_t, outside, ignored)
        ctx.input_dtype = logits.dtype
        return loss

    @staticmethod
    def backward(ctx: Any, grad_output: Tensor):
        softmax, local_t, outside, ignored = ctx.saved_tensors
        g = softmax.clone()
        g2 = g.reshape(-1, g.shape[-1])
        rows = torch.arange(g2.shape[0])
        g2[rows, local_t.reshape(-1)] -= (~outside.reshape(-1)).to(g2.dtype)
        g = g2.reshape_as(g)
        g.masked_fill_(ignored.unsqueeze(-1), 0.0)
        grad = g * grad_output.to(g.dtype).unsqueeze(-1)
        return grad.to(ctx.input_dtype), None, None


def cross_entropy_tokens(
    logits: Tensor, targets: Tensor, ignore_index: int = -100, reduction: str = "none"
) -> Tensor:
    """``VocabParallelCrossEntropy.forward`` (tensor_parallel/cross_entropy.py:108-123)."""
    if logits.shape[:-1] != targets.shape:
        raise ValueError("targets must match all non-vocabulary logits dimensions")
    invalid = (targets != ignore_index) & ((targets < 0) | (targets >= logits.shape[-1]))
    if torch.any(invalid):
        raise ValueError("targets contain ids outside the original (unpadded) vocabulary")
    loss = _TokenCrossEntropy.apply(logits, targets, ignore_index)
    if reduction == "none":
        return loss
    if reduction == "sum":
        return loss.sum()
    valid = (targets != ignore_index).sum().clamp_min(1)
    return loss.sum() / valid


# ---------------------------------------------------------------- modules
class _ProjectedLinear(nn.Module):
    """Column/RowParallelLinear at TP=1: ``self.linear = nn.Linear``
    (tensor_parallel/layers.py:56-62).  With a bias, the column form keeps it in
    the ``nn.Linear`` (its default init); the row form keeps a zero-initialised
    ``self.bias`` beside a bias-free ``nn.Linear`` and adds it after the product
    (layers.py:110-126, 153-155)."""

    def __init__(self, in_features: int, out_features: int, dtype: torch.dtype | None, *,
                 bias: bool = False, row: bool = False) -> None:
        super().__init__()
        self.linear = nn.Linear(in_features, out_features, bias=bias and not row, dtype=dtype)
        self.bias = nn.Parameter(torch.zeros(out_features, dtype=dtype)) if bias and row else None

    def forward(self, x: Tensor) -> Tensor:
        y = self.linear(x)
        return y + self.bias if self.bias is not None else y


class OracleAttention(nn.Module):
    """GPTAttention (models/gpt/attention.py:35-209) at TP=CP=1."""

    def __init__(self, config: Any, dtype: torch.dtype | None = None) -> None:
        super().__init__()
        self.hidden_size = int(_cfg(config, "hidden_size"))
        self.num_heads = int(_cfg(config, "heads", "num_attention_heads"))
        self.num_kv_heads = int(_cfg(config, "num_kv_heads", "kv_heads", default=self.num_heads))
        self.head_dim = self.hidden_size // self.num_heads
        kv_hidden = self.num_kv_heads * self.head_dim
        bias = bool(_cfg(config, "linear_bias", "bias", default=False))  # attention.py:78-117
        self.q_proj = _ProjectedLinear(self.hidden_size, self.hidden_size, dtype, bias=bias)
        self.k_proj = _ProjectedLinear(self.hidden_size, kv_hidden, dtype, bias=bias)
        self.v_proj = _ProjectedLinear(self.hidden_size, kv_hidden, dtype, bias=bias)
        self.out_proj = _ProjectedLinear(self.hidden_size, self.hidden_size, dtype, bias=bias, row=True)
        self.rope = OracleRotaryEmbedding(self.head_dim, float(_cfg(config, "rope_theta", default=1e4)))
        self.dropout = float(_cfg(config, "attention_dropout", "dropout", default=0.0))

    def forward(self, x: Tensor, *, position_ids: Tensor, sequence_offset: int = 0,
                dropout_seed: int = 0) -> Tensor:
        b, s, _ = x.shape
        q = self.q_proj(x).view(b, s, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(x).view(b, s, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(x).view(b, s, self.num_kv_heads, self.head_dim).transpose(1, 2)
        cos, sin = self.rope(position_ids, dtype=q.dtype)
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        # attention.py:190-206: dropout_p only in training
        ctx = local_attention(q, k, v, causal=True, sequence_offset=sequence_offset,
                              dropout_p=self.dropout if self.training else 0.0, dropout_seed=dropout_seed)
        ctx = ctx.transpose(1, 2).contiguous().view(b, s, self.hidden_size)
        return self.out_proj(ctx)


class OracleMLP(nn.Module):
    """GPTMLP (models/gpt/mlp.py:22-78)."""

    def __init__(self, config: Any, dtype: torch.dtype | None = None) -> None:
        super().__init__()
        h = int(_cfg(config, "hidden_size"))
        f = int(_cfg(config, "ffn_hidden_size"))
        bias = bool(_cfg(config, "linear_bias", "bias", default=False))  # mlp.py:40-70
        self.gate_proj = _ProjectedLinear(h, f, dtype, bias=bias)
        self.up_proj = _ProjectedLinear(h, f, dtype, bias=bias)
        self.down_proj = _ProjectedLinear(f, h, dtype, bias=bias, row=True)

    def forward(self, x: Tensor) -> Tensor:
        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x)))


class OracleLayer(nn.Module):
    """GPTLayer (models/gpt/layer.py:22-137): pre-norm attention + SwiGLU with
    residuals, each residual branch through dropout in training (:114-137).
    ``dropout_seed(layer, op)`` gives the mask key of each random op ("attention.tp=0",
    "attention_residual", "mlp_residual")."""

    def __init__(self, config: Any, layer_index: int, dtype: torch.dtype | None = None) -> None:
        super().__init__()
        eps = float(_cfg(config, "norm_epsilon", "norm_eps", "rms_norm_eps", default=1e-6))
        h = int(_cfg(config, "hidden_size"))
        self.layer_index = layer_index
        self.input_norm = OracleRMSNorm(h, eps, dtype)
        self.attention = OracleAttention(config, dtype)
        self.post_attention_norm = OracleRMSNorm(h, eps, dtype)
        self.mlp = OracleMLP(config, dtype)
        self.dropout = float(_cfg(config, "hidden_dropout", "dropout", default=0.0))
        self.forward_calls = 0

    def _residual(self, residual: Tensor, branch: Tensor, seed: int) -> Tensor:
        if not self.training or self.dropout == 0.0:
            return residual + branch
        return dropout_add(branch, self.dropout, seed, residual=residual)

    def forward(self, x: Tensor, *, position_ids: Tensor, sequence_offset: int = 0,
                dropout_seed: Any = None) -> Tensor:
        self.forward_calls += 1
        seed = dropout_seed if dropout_seed is not None else (lambda layer, op: 0)
        a = self.attention(self.input_norm(x), position_ids=position_ids, sequence_offset=sequence_offset,
                           dropout_seed=seed(self.layer_index, "attention.tp=0"))
        h = self._residual(x, a, seed(self.layer_index, "attention_residual"))
        return self._residual(h, self.mlp(self.post_attention_norm(h)), seed(self.layer_index, "mlp_residual"))


@dataclass
class GPTOutput:
    """models/gpt/model.py:31-37."""

    logits: Tensor | None
    loss: Tensor | None
    hidden_states: Tensor


def embedding_lookup(input_ids: Tensor, weight: Tensor) -> Tensor:
    """``VocabParallelEmbedding.forward`` at TP=1 (tensor_parallel/embedding.py:60-68).

    The partition is the whole table [0, V): ids outside it are replaced by 0
    for the gather and their rows masked to zero afterwards, so they read
    nothing and pass no gradient to the table.
    """
    if input_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"input_ids must be an integer tensor, got {input_ids.dtype}")
    outside = (input_ids < 0) | (input_ids >= weight.shape[0])
    local_ids = input_ids.masked_fill(outside, 0)
    return F.embedding(local_ids, weight).masked_fill(outside.unsqueeze(-1), 0.0)


class _Embedding(nn.Module):
    """VocabParallelEmbedding at TP=1 (tensor_parallel/embedding.py:22-75): N(0, init_std)."""

    def __init__(self, vocab: int, hidden: int, init_std: float, dtype: torch.dtype | None) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.empty(vocab, hidden, dtype=dtype))
        nn.init.normal_(self.weight, mean=0.0, std=init_std)

    def forward(self, input_ids: Tensor) -> Tensor:
        return embedding_lookup(input_ids, self.weight)


class _LMHead(nn.Module):
    """VocabParallelLinear (tensor_parallel/layers.py:158-214): the embedding's
    weight when tied, else its own N(0, init_std) weight."""

    def __init__(self, weight: nn.Parameter) -> None:
        super().__init__()
        self.weight = weight

    def forward(self, x: Tensor) -> Tensor:
        return F.linear(x, self.weight)


class OracleGPTModel(nn.Module):
    """GPTModel (models/gpt/model.py:40-250) on one rank.

    Construction order equals the reference's, so ``torch.manual_seed(s)``
    before construction yields the reference's initial weights: embedding
    N(0, 0.02) first (model.py:86-98), then per layer the seven ``nn.Linear``
    kaiming-uniform inits in q, k, v, out, gate, up, down order
    (attention.py:82-117, mlp.py:44-70), norms at ones.

    ``activation_checkpoint_config.mode == "full"`` wraps each layer with
    ``layer_index % block_interval == 0`` in non-reentrant
    ``torch.utils.checkpoint`` with ``preserve_rng_state=True``
    (model.py:162-170, 215-233; nn/activation_checkpoint.py:73-100).
    """

    def __init__(
        self,
        config: Any,
        *,
        activation_checkpoint_config: Any | None = None,
        dtype: torch.dtype | None = None,
        dropout_seed: Any = None,
    ) -> None:
        super().__init__()
        self.config = config
        self.activation_checkpoint_config = activation_checkpoint_config
        # dropout (models/gpt/model.py:72, 203-212; layer.py:114-137; attention.py:190-206):
        # dropout_seed(layer, op) keys each random op's mask
        self.dropout = float(_cfg(config, "embedding_dropout", "dropout", default=0.0))
        self.dropout_seed = dropout_seed if dropout_seed is not None else (lambda layer, op: 0)
        h = int(_cfg(config, "hidden_size"))
        layers = int(_cfg(config, "layers", "num_layers"))
        vocab = int(_cfg(config, "vocab_size"))
        init_std = float(_cfg(config, "init_std", default=0.02))
        eps = float(_cfg(config, "norm_epsilon", "norm_eps", "rms_norm_eps", default=1e-6))
        self.embedding = _Embedding(vocab, h, init_std, dtype)
        self.layers = nn.ModuleList([OracleLayer(config, i, dtype) for i in range(layers)])
        self.final_norm = OracleRMSNorm(h, eps, dtype)
        if bool(_cfg(config, "tie_embeddings", default=True)):  # model.py:125-142
            self.lm_head = _LMHead(self.embedding.weight)
        else:
            head = nn.Parameter(torch.empty(vocab, h, dtype=dtype))
            nn.init.normal_(head, mean=0.0, std=init_std)
            self.lm_head = _LMHead(head)

    def _checkpoint_layer(self, layer: OracleLayer) -> bool:
        cfg = self.activation_checkpoint_config
        if cfg is None or str(getattr(cfg, "mode", "none")) != "full" or not self.training:
            return False
        interval = int(getattr(cfg, "block_interval", 1))
        if interval <= 0:
            raise ValueError("activation checkpoint block_interval must be positive")
        return layer.layer_index % interval == 0

    def forward(self, input_ids: Tensor, *, labels: Tensor | None = None,
                position_ids: Tensor | None = None) -> GPTOutput:
        """model.py:171-250 at CP=TP=1: default positions arange(S) with offset 0,
        else the given ids with offset position_ids[0] (:193-200), passed to every
        layer as RoPE positions and the causal mask's query offset."""
        hidden = self.embedding(input_ids)
        seq = input_ids.shape[1]
        if position_ids is None:
            offset = 0
            position_ids = torch.arange(0, seq)
        else:
            offset = int(position_ids.reshape(-1)[0].item())
        if self.training and self.dropout:
            hidden = dropout_add(hidden, self.dropout, self.dropout_seed(0, "embedding"))
        for layer in self.layers:
            if self._checkpoint_layer(layer):
                hidden = torch_checkpoint(
                    lambda x, cur=layer: cur(x, position_ids=position_ids, sequence_offset=offset,
                                             dropout_seed=self.dropout_seed),
                    hidden,
                    use_reentrant=False,
                    preserve_rng_state=True,
                )
            else:
                hidden = layer(hidden, position_ids=position_ids, sequence_offset=offset,
                               dropout_seed=self.dropout_seed)
        hidden = self.final_norm(hidden)
        logits = self.lm_head(hidden)
        loss = None
        if labels is not None:
            loss = cross_entropy_tokens(logits, labels, reduction="mean")
        return GPTOutput(logits=logits, loss=loss, hidden_states=hidden)


# ---------------------------------------------------------------- optimizer
@torch.no_grad()
def clip_coefficient(total_norm: Tensor, max_norm: float) -> Tensor:
    """``clamp(max_norm / (norm + 1e-6), max=1)`` (data_parallel/_zero.py:160-163)."""
    return torch.clamp(max_norm / (total_norm + 1.0e-6), max=1.0)


@torch.no_grad()
def adamw_master_step(
    master: Tensor,
    exp_avg: Tensor,
    exp_avg_sq: Tensor,
    grad: Tensor,
    *,
    step: int,
    lr: float,
    betas: tuple[float, float] = (0.9, 0.95),
    eps: float = 1.0e-8,
    weight_decay: float = 0.0,
) -> None:
    """fp32-master AdamW on flat shards (data_parallel/_zero.py:166-199), in place.

    ``m = b1 m + (1-b1) g``; ``v = b2 v + (1-b2) g^2``; decoupled decay
    ``p *= 1 - lr wd``; ``p -= (lr / bc1) * m / (sqrt(v) / sqrt(bc2) + eps)``.
    """
    beta1, beta2 = betas
    bc1 = 1.0 - beta1**step
    bc2 = 1.0 - beta2**step
    step_size = lr / bc1
    g = grad.float()
    exp_avg.mul_(beta1).add_(g, alpha=1.0 - beta1)
    exp_avg_sq.mul_(beta2).addcmul_(g, g, value=1.0 - beta2)
    if weight_decay:
        master.mul_(1.0 - lr * weight_decay)
    denom = exp_avg_sq.sqrt().div_(bc2**0.5).add_(eps)
    master.addcdiv_(exp_avg, denom, value=-step_size)
