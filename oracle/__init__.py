"""CPU oracle for the activation-checkpointed GPT block (TEST INFRASTRUCTURE ONLY).

This package restates, in plain PyTorch on the CPU, the arithmetic of the
reference's hot path (pyy233/Nano-Megatron, ``src/nano_megatron``): RMSNorm,
RoPE, SwiGLU MLP, MHA/GQA causal attention (local and ring-share maths), the
tied-embedding LM head with vocabulary cross entropy, the per-layer activation
checkpoint switch, and the fp32-master AdamW step.  Every function cites the
reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or as the timed
CPU baseline).  The product package ``nano_megatron_amd`` never imports it and
has no CPU fallback.

Each function is pinned by an independent check in ``tests/test_oracle.py``:
PyTorch library routines that implement the same textbook definition
(``F.rms_norm``, ``F.scaled_dot_product_attention``, ``F.cross_entropy``,
``torch.optim.AdamW``), closed-form derivatives, fp64 brute force on tiny
inputs, and invariants (RoPE norm preservation and exact inversion, causality,
GQA == repeat_interleave, checkpointed == eager gradients).
"""

from oracle.reference import (  # noqa: F401
    GPTOutput,
    OracleAttention,
    OracleGPTModel,
    OracleLayer,
    OracleMLP,
    OracleRMSNorm,
    OracleRotaryEmbedding,
    adamw_master_step,
    apply_rotary_pos_emb,
    cross_entropy_tokens,
    local_attention,
    ring_attention_backward,
    ring_attention_forward,
    rms_norm,
    rope_cos_sin,
    swiglu,
)
