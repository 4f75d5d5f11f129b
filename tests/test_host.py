"""Host-side logic on the CPU: configs, the backend seam, module structure and
the no-fallback rule (the kernels refuse CPU tensors)."""

from __future__ import annotations

import pytest
import torch

import nano_megatron_amd as nm
from nano_megatron_amd import functional as Fn


def test_configs_validate_like_the_reference() -> None:
    cfg = nm.GPTConfig(layers=24, hidden_size=1024, ffn_hidden_size=2736, heads=16, seq_length=512,
                       vocab_size=8192)
    assert cfg.num_kv_heads == 16 and cfg.head_dim == 64
    with pytest.raises(ValueError):
        nm.GPTConfig(hidden_size=100, heads=12)
    with pytest.raises(ValueError):
        nm.GPTConfig(heads=12, kv_heads=5)
    assert nm.ActivationCheckpointConfig(mode="full").block_interval == 1
    with pytest.raises(ValueError, match="non-reentrant"):
        nm.ActivationCheckpointConfig(use_reentrant=True)
    with pytest.raises(ValueError):
        nm.ActivationCheckpointConfig(mode="sometimes")
    with pytest.raises(ValueError):
        nm.ActivationCheckpointConfig(selective_ops=("norm",))
    with pytest.raises(ValueError):
        nm.KernelConfig(backend="torch")


def test_build_kernel_backend_selects_hip() -> None:
    backend = nm.build_kernel_backend(nm.KernelConfig())
    assert isinstance(backend, nm.HipKernelBackend) and backend.name == "hip"
    assert isinstance(nm.build_kernel_backend("hip"), nm.HipKernelBackend)
    with pytest.raises(ValueError, match="unknown kernel backend"):
        nm.build_kernel_backend("cuda")
    lin = backend.linear(8, 4, bias=False)
    assert tuple(lin.weight.shape) == (4, 8) and lin.bias is None
    norm = backend.rms_norm(8, 1e-5)
    assert torch.equal(norm.weight, torch.ones(8))


def test_local_attention_validates_like_the_reference() -> None:
    backend = nm.HipKernelBackend()
    q = torch.randn(1, 6, 4, 8)
    with pytest.raises(ValueError, match="divisible by KV heads"):
        backend.local_attention(q, torch.randn(1, 4, 4, 8), torch.randn(1, 4, 4, 8))
    with pytest.raises(ValueError, match="identical shapes"):
        backend.local_attention(q, torch.randn(1, 2, 4, 8), torch.randn(1, 2, 5, 8))
    for p in (-0.1, 1.0):
        with pytest.raises(ValueError, match="dropout probability"):
            backend.local_attention(q, torch.randn(1, 2, 4, 8), torch.randn(1, 2, 4, 8), dropout_p=p)
    with pytest.raises(ValueError, match="no CPU fallback"):
        backend.local_attention(q, torch.randn(1, 2, 4, 8), torch.randn(1, 2, 4, 8), dropout_p=0.1)


def test_kernels_refuse_cpu_tensors() -> None:
    x = torch.randn(4, 64)
    with pytest.raises(ValueError, match="no CPU fallback"):
        nm.rms_norm(x, torch.ones(64), 1e-5)
    with pytest.raises(ValueError, match="no CPU fallback"):
        nm.swiglu(x, x)
    q = torch.randn(1, 2, 4, 64)
    with pytest.raises(ValueError, match="no CPU fallback"):
        nm.attention(q, q, q)
    with pytest.raises(ValueError, match="no CPU fallback"):
        nm.lm_head_cross_entropy(torch.randn(2, 3, 64), torch.randn(16, 64),
                                 torch.zeros(2, 3, dtype=torch.long))


def test_captured_step_refuses_cpu_tensors() -> None:
    from nano_megatron_amd.graph import CapturedTrainStep

    x = torch.zeros(2, 8, dtype=torch.long)
    with pytest.raises(ValueError, match="GPU"):
        CapturedTrainStep(torch.nn.Linear(2, 2), None, x, x)


def test_target_check_rules() -> None:
    """The cross entropy's target-range rule (tensor_parallel/cross_entropy.py:
    109-114): ids in [0, vocab) or ignore_index pass; anything else raises."""
    from nano_megatron_amd import functional as Fn

    ok = torch.tensor([[0, 15, -100], [3, 7, 1]])
    Fn.TargetCheck(ok, 16).raise_if_invalid()
    Fn.TargetCheck(torch.tensor([[-1, 3]]), 16, ignore_index=-1).raise_if_invalid()
    for bad in (16, -5, -100):
        t = ok.clone()
        t[1, 2] = bad
        check = Fn.TargetCheck(t, 16, ignore_index=-100 if bad != -100 else -1)
        with pytest.raises(ValueError, match="outside the original"):
            check.raise_if_invalid()


def test_model_structure_matches_reference_keys_and_rejects_parallel() -> None:
    cfg = nm.GPTConfig(layers=2, hidden_size=64, ffn_hidden_size=96, heads=2, kv_heads=1,
                       seq_length=16, vocab_size=128)
    model = nm.GPTModel(cfg)
    keys = set(model.state_dict())
    for k in ("embedding.weight", "lm_head.weight", "final_norm.weight",
              "layers.1.attention.k_proj.linear.weight", "layers.0.mlp.down_proj.linear.weight",
              "layers.0.post_attention_norm.weight"):
        assert k in keys
    assert model.lm_head.weight is model.embedding.weight
    assert tuple(model.layers[0].attention.k_proj.weight.shape) == (32, 64)
    assert all(layer.fusable() for layer in model.layers)

    class _Group:
        size = 2

    class _Parallel:
        tp = _Group()

    with pytest.raises(ValueError, match="one GPU"):
        nm.GPTModel(cfg, parallel=_Parallel())
    with pytest.raises(ValueError, match="no CPU fallback"):
        model(torch.zeros(1, 16, dtype=torch.long))


def test_rope_tables_from_reference_cos_sin_layout() -> None:
    cos = torch.randn(5, 8)
    ct, st, pos = Fn.rope_tables_from_cos_sin(cos, cos, 2, 5)
    assert ct.shape == (5, 4) and pos.dtype == torch.int32 and pos.tolist() == list(range(5))
    ct, st, pos = Fn.rope_tables_from_cos_sin(torch.randn(2, 5, 8), torch.randn(2, 5, 8), 2, 5)
    assert ct.shape == (10, 4) and pos.shape == (2, 5) and pos[1, 0].item() == 5
    with pytest.raises(ValueError):
        Fn.rope_tables_from_cos_sin(torch.randn(8), torch.randn(8), 1, 8)
