"""Config blocks the hot path reads, mirroring the reference's frozen dataclasses.

GPTConfig follows config/schema.py:205-273, ActivationCheckpointConfig
config/schema.py:381-416, KernelConfig config/schema.py:298-307 (the
reference's enum has only "torch"; this package adds "hip").  Validation
raises the same exception types as the reference.
"""

from __future__ import annotations

from dataclasses import dataclass

CHECKPOINT_MODES = ("none", "full", "selective")
KERNEL_BACKENDS = ("hip",)


def _require_int(name: str, value, minimum: int = 1) -> None:
    if isinstance(value, bool) or not isinstance(value, int):
        raise TypeError(f"{name} must be an integer")
    if value < minimum:
        raise ValueError(f"{name} must be >= {minimum}, got {value}")


def _require_positive(name: str, value) -> None:
    if isinstance(value, bool) or not isinstance(value, (int, float)) or value <= 0:
        raise ValueError(f"{name} must be a positive number, got {value!r}")


@dataclass(frozen=True)
class GPTConfig:
    """config/schema.py:205-273 (defaults included)."""

    layers: int = 12
    hidden_size: int = 768
    ffn_hidden_size: int = 2048
    heads: int = 12
    kv_heads: int | None = None
    seq_length: int = 2048
    vocab_size: int = 50304
    rope_theta: float = 10000.0
    dropout: float = 0.0
    tie_embeddings: bool = True
    norm_epsilon: float = 1.0e-5
    bias: bool = False

    def __post_init__(self) -> None:
        for name in ("layers", "hidden_size", "ffn_hidden_size", "heads", "seq_length", "vocab_size"):
            _require_int(f"model.{name}", getattr(self, name))
        if self.kv_heads is not None:
            _require_int("model.kv_heads", self.kv_heads)
        _require_positive("model.rope_theta", self.rope_theta)
        _require_positive("model.norm_epsilon", self.norm_epsilon)
        if isinstance(self.dropout, bool) or not 0 <= self.dropout < 1:
            raise ValueError(f"model.dropout must be in [0, 1), got {self.dropout}")
        if self.hidden_size % self.heads:
            raise ValueError(
                f"model.hidden_size ({self.hidden_size}) must be divisible by model.heads ({self.heads})"
            )
        if self.num_kv_heads > self.heads or self.heads % self.num_kv_heads:
            raise ValueError(
                "model.kv_heads must divide model.heads and cannot exceed it; "
                f"got heads={self.heads}, kv_heads={self.num_kv_heads}"
            )

    @property
    def num_layers(self) -> int:
        return self.layers

    @property
    def num_attention_heads(self) -> int:
        return self.heads

    @property
    def num_kv_heads(self) -> int:
        return self.heads if self.kv_heads is None else self.kv_heads

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.heads


@dataclass(frozen=True)
class ActivationCheckpointConfig:
    """config/schema.py:381-416: mode none|full|selective, non-reentrant only."""

    mode: str = "none"
    block_interval: int = 1
    selective_ops: tuple[str, ...] = ("attention", "mlp")
    use_reentrant: bool = False
    offload_saved_tensors: bool = False

    def __post_init__(self) -> None:
        mode = getattr(self.mode, "value", self.mode)
        if mode not in CHECKPOINT_MODES:
            raise ValueError(f"activation_checkpoint.mode must be one of {CHECKPOINT_MODES}, got {mode!r}")
        object.__setattr__(self, "mode", mode)
        object.__setattr__(self, "selective_ops", tuple(self.selective_ops))
        _require_int("activation_checkpoint.block_interval", self.block_interval)
        if not self.selective_ops:
            raise ValueError("activation_checkpoint.selective_ops cannot be empty")
        unknown = set(self.selective_ops) - {"attention", "mlp"}
        if unknown:
            raise ValueError(
                "activation_checkpoint.selective_ops contains unsupported values: "
                + ", ".join(sorted(unknown))
            )
        if self.use_reentrant:
            raise ValueError("Nano-Megatron only supports non-reentrant activation checkpointing")


@dataclass(frozen=True)
class KernelConfig:
    """config/schema.py:298-307 with the "hip" backend."""

    backend: str = "hip"

    def __post_init__(self) -> None:
        backend = getattr(self.backend, "value", self.backend)
        if backend not in KERNEL_BACKENDS:
            raise ValueError(f"kernels.backend must be one of {KERNEL_BACKENDS}, got {backend!r}")
        object.__setattr__(self, "backend", backend)
