"""MI355X-native activation-checkpointed GPT block for pyy233/Nano-Megatron.

The package mirrors the reference's hot-path API (``nano_megatron.nn``,
``nano_megatron.nn.kernels``, ``nano_megatron.models.gpt``) on top of
``libnmb.so``, the gfx950 HIP kernels declared in ``include/nmb.h``.  It runs
on one GPU and has no CPU fallback.
"""

from nano_megatron_amd.config import (
    ActivationCheckpointConfig,
    GPTConfig,
    KernelConfig,
)
from nano_megatron_amd.functional import (
    attention,
    lm_head_cross_entropy,
    ring_attention,
    rms_norm,
    swiglu,
)
from nano_megatron_amd.gpt import (
    DenseGPTComponents,
    GPTAttention,
    GPTLayer,
    GPTMLP,
    GPTModel,
    GPTOutput,
)
from nano_megatron_amd.kernels import HipKernelBackend, KernelBackend, build_kernel_backend
from nano_megatron_amd.train import StepOutput, train_step
from nano_megatron_amd.nn import (
    ActivationCheckpoint,
    RMSNorm,
    RotaryEmbedding,
    activation_checkpoint,
    activation_rng_context,
    apply_rotary_pos_emb,
    parallel_dropout,
)

__all__ = [
    "ActivationCheckpointConfig",
    "DenseGPTComponents",
    "GPTAttention",
    "GPTConfig",
    "GPTLayer",
    "GPTMLP",
    "GPTModel",
    "GPTOutput",
    "HipKernelBackend",
    "KernelBackend",
    "KernelConfig",
    "RMSNorm",
    "RotaryEmbedding",
    "activation_checkpoint",
    "activation_rng_context",
    "parallel_dropout",
    "ActivationCheckpoint",
    "StepOutput",
    "train_step",
    "apply_rotary_pos_emb",
    "attention",
    "build_kernel_backend",
    "lm_head_cross_entropy",
    "ring_attention",
    "rms_norm",
    "swiglu",
]
