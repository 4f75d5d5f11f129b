"""The kernel-backend seam with the MI355X backend behind it.

Mirrors nn/kernels/interface.py:10-25 (the ``KernelBackend`` protocol) and
nn/kernels/__init__.py:11-22 (``build_kernel_backend``).  ``HipKernelBackend``
is the drop-in for ``TorchKernelBackend`` (nn/kernels/torch_backend.py:14-76):
same members, argument meanings and exceptions.
"""

from __future__ import annotations

from typing import Any, Protocol

from torch import Tensor, nn

from nano_megatron_amd import functional as Fn
from nano_megatron_amd.nn import RMSNorm


class KernelBackend(Protocol):
    name: str

    def linear(self, in_features: int, out_features: int, **kwargs: Any) -> nn.Module: ...

    def rms_norm(self, hidden_size: int, eps: float, **kwargs: Any) -> nn.Module: ...

    def local_attention(self, q: Tensor, k: Tensor, v: Tensor, **kwargs: Any) -> Tensor: ...


class Linear(nn.Linear):
    """``nn.Linear`` (same parameters, attribute names and kaiming-uniform init,
    so seeded weights equal the reference's) whose product runs on this
    library's GEMM kernels (bf16 and fp32 MFMA) instead of the vendor GEMM."""

    def forward(self, x: Tensor) -> Tensor:
        return Fn.linear(x, self.weight, self.bias)


class HipKernelBackend:
    """gfx950 kernels: MFMA GEMMs for ``linear``, fused RMSNorm, MFMA attention."""

    name = "hip"

    def linear(self, in_features: int, out_features: int, **kwargs: Any) -> nn.Module:
        return Linear(in_features, out_features, **kwargs)

    def rms_norm(self, hidden_size: int, eps: float, **kwargs: Any) -> nn.Module:
        return RMSNorm(hidden_size, eps, **kwargs)

    def local_attention(
        self,
        q: Tensor,
        k: Tensor,
        v: Tensor,
        *,
        causal: bool = True,
        sequence_offset: int = 0,
        dropout_p: float = 0.0,
        scale: float | None = None,
        attention_mask: Tensor | None = None,
        **_: Any,
    ) -> Tensor:
        """Attention for [B,H,S,D] tensors; GQA reads KV heads in place (no repeat)."""
        if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
            raise ValueError("q, k and v must have [batch, heads, sequence, head_dim] shape")
        if k.shape != v.shape:
            raise ValueError("k and v must have identical shapes")
        if q.shape[0] != k.shape[0] or q.shape[-1] != k.shape[-1]:
            raise ValueError("q and k/v must agree on batch size and head_dim")
        if q.shape[1] % k.shape[1]:
            raise ValueError(
                f"query heads ({q.shape[1]}) must be divisible by KV heads ({k.shape[1]})"
            )
        if attention_mask is not None or dropout_p:
            # the seed comes from torch's default CPU generator, the stream the
            # caller's activation_rng_context forks (models/gpt/attention.py:190-206)
            return Fn.masked_attention(q, k, v, attention_mask, causal=causal,
                                       sequence_offset=sequence_offset, scale=scale, dropout_p=dropout_p)
        return Fn.attention(q, k, v, causal=causal, sequence_offset=sequence_offset, scale=scale)


def build_kernel_backend(config: Any, parallel: Any = None) -> KernelBackend:
    """nn/kernels/__init__.py:11-22 with the "hip" value."""
    del parallel
    backend = getattr(config, "backend", config)
    value = getattr(backend, "value", backend)
    if value == "hip":
        return HipKernelBackend()
    raise ValueError(f"unknown kernel backend: {value!r}")
