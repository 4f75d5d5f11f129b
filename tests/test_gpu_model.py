"""End-to-end parity of the fused checkpointed block model on the GPU.

* Config 1 (fp32): 4 layers, hidden 256, 4 heads, ffn 688, vocab 8192 tied,
  B4 S128 from seed 0, full recompute, AdamW lr 3e-4 for 5 steps: loss every
  step and every gradient against the oracle, rtol 1e-5 with atol 1e-5 of
  each tensor's largest magnitude and a relative L2 error within 1e-5.
* bf16 (MHA and GQA, 2 layers; config 3's 24 layers at B1 S512; config 4's
  16 layers at B1 S2048): loss within rtol 1e-3 and every gradient within
  the bf16 bar of tests/parity.py (relative L2 error against the fp32
  evaluation of the same bf16 weights at most 1.5x the oracle's own bf16
  error + 5e-3).
* The recomputed forward is bit-identical to the original forward, and the
  full-recompute gradients are bit-identical to the no-checkpoint gradients.
"""

from __future__ import annotations

import pytest
import torch

import nano_megatron_amd as nm
from nano_megatron_amd import block as B
from oracle import reference as R
from parity import assert_bf16_grad, assert_bf16_grads, assert_close_scaled, assert_grads_scaled, assert_loss_close

pytestmark = pytest.mark.gpu


def c1_config(**kw):
    base = dict(layers=4, hidden_size=256, ffn_hidden_size=688, heads=4, seq_length=128,
                vocab_size=8192, norm_epsilon=1e-5, rope_theta=1e4)
    base.update(kw)
    return nm.GPTConfig(**base)


def c1_batch():
    g = torch.Generator().manual_seed(0)
    ids = torch.randint(0, 8192, (4, 129), generator=g)
    return ids[:, :128].contiguous(), ids[:, 1:].contiguous()


def build_pair(cfg, mode, dtype, device, seed=0):
    """This build's model and the oracle's with the same weights; in bf16 also
    the oracle in fp32 on those bf16 weights (the exact result the bf16 bar
    measures both against), else None."""
    ck = nm.ActivationCheckpointConfig(mode=mode)
    torch.manual_seed(seed)
    ours = nm.GPTModel(cfg, activation_checkpoint_config=ck).to(device=device, dtype=dtype)
    state = {k: v.cpu() for k, v in ours.state_dict().items()}
    torch.manual_seed(seed)
    ref = R.OracleGPTModel(cfg, activation_checkpoint_config=ck).to(dtype=dtype)
    ref.load_state_dict(state)
    ours.train()
    ref.train()
    ref32 = None
    if dtype != torch.float32:
        ref32 = R.OracleGPTModel(cfg, activation_checkpoint_config=ck)
        ref32.load_state_dict({k: v.float() for k, v in state.items()})
        ref32.train()
    return ours, ref, ref32


def check_model(ours, ref, ref32, dtype, ids, labels, device, **kw):
    """Loss and every gradient of one forward/backward of ``ours`` on the GPU
    against the oracle (and, in bf16, the fp32 oracle) on the CPU."""
    dev = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
    lo = ours(ids.to(device), labels=labels.to(device), **dev).loss
    lo.backward()
    lr = ref(ids, labels=labels, **kw).loss
    lr.backward()
    assert_loss_close(lo, lr, dtype)
    if ref32 is None:
        assert_grads_scaled(ours, ref, dtype)
    else:
        ref32(ids, labels=labels, **kw).loss.backward()
        assert_bf16_grads(ours, ref, ref32)
    return lo, lr


def test_config1_fp32_five_adamw_steps_match_oracle(device) -> None:
    """Five AdamW steps (lr 3e-4, betas (0.9, 0.95), eps 1e-8, weight decay
    0.1): at every step, from the same weights, the loss and every gradient
    within the fp32 bar.  Each step starts the oracle from this build's
    weights: AdamW's first updates are about lr * sign(grad), so gradients
    that differ by fp32 rounding near zero move weights by up to 2 lr apart,
    and two trajectories drift apart by more than any rounding bar after one
    step (the embedding gradient by 1.1e-5 relative at step 1)."""
    cfg = c1_config()
    ours, ref, _ = build_pair(cfg, "full", torch.float32, device)
    ids, labels = c1_batch()
    opt_o = torch.optim.AdamW(ours.parameters(), lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    losses = []
    for step in range(5):
        ref.load_state_dict({k: v.cpu() for k, v in ours.state_dict().items()})
        opt_o.zero_grad(set_to_none=True)
        ref.zero_grad(set_to_none=True)
        lo = ours(ids.to(device), labels=labels.to(device)).loss
        lr = ref(ids, labels=labels).loss
        lo.backward()
        lr.backward()
        assert_loss_close(lo, lr, torch.float32, msg=f"loss step {step}")
        assert_grads_scaled(ours, ref, torch.float32)
        opt_o.step()
        losses.append(float(lo.detach()))
    assert losses[-1] < losses[0]  # the steps train


@pytest.mark.parametrize("kv_heads,mode", [(None, "full"), (2, "full"), (None, "none"), (2, "selective")])
def test_bf16_model_matches_oracle(device, kv_heads, mode) -> None:
    cfg = c1_config(layers=2, kv_heads=kv_heads)
    ours, ref, ref32 = build_pair(cfg, mode, torch.bfloat16, device)
    ids, labels = c1_batch()
    labels[0, :5] = -100
    check_model(ours, ref, ref32, torch.bfloat16, ids, labels, device)


def _block_inputs(device, dtype=torch.bfloat16, b=4, s=256, h=512, heads=8, kv=4, f=1376):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(b, s, h, generator=g).to(dtype).to(device)
    w = (
        1 + 0.1 * torch.randn(h, generator=g),
        0.02 * torch.randn(h, h, generator=g),
        0.02 * torch.randn(kv * h // heads, h, generator=g),
        0.02 * torch.randn(kv * h // heads, h, generator=g),
        0.02 * torch.randn(h, h, generator=g),
        1 + 0.1 * torch.randn(h, generator=g),
        0.02 * torch.randn(f, h, generator=g),
        0.02 * torch.randn(f, h, generator=g),
        0.02 * torch.randn(h, f, generator=g),
    )
    w = tuple(t.to(dtype).to(device) for t in w)
    tab = nm.RotaryEmbedding(h // heads).tables(device, s)
    meta = B.BlockMeta(heads=heads, kv_heads=kv, head_dim=h // heads, eps=1e-5, sequence_offset=0,
                       cos=tab.cos, sin=tab.sin, positions=None)
    return x, w, meta


def test_recompute_is_bit_identical_to_forward(device) -> None:
    x, w, meta = _block_inputs(device)
    with torch.no_grad():
        fwd = B.block_forward(x, w, meta, recompute=False)
        rec = B.block_forward(x, w, meta, recompute=True)
    for key in ("n1", "qkv", "o2", "lse", "h", "n2", "gu"):
        assert torch.equal(fwd[key], rec[key]), key


def test_full_recompute_grads_bit_identical_to_eager(device) -> None:
    x, w, meta = _block_inputs(device)
    dy = torch.randn_like(x)
    results = []
    for fn in (B.CheckpointedBlockFunction, B.EagerBlockFunction, "offload"):
        xs = x.clone().requires_grad_(True)
        ws = [t.clone().requires_grad_(True) for t in w]
        if fn is B.EagerBlockFunction:
            y = fn.apply(xs, meta, *ws)
        else:
            y = B.CheckpointedBlockFunction.apply(xs, meta, fn == "offload", *ws)
        y.backward(dy)
        results.append((y.detach(), xs.grad, *[t.grad for t in ws]))
    for other in results[1:]:
        for a, b in zip(results[0], other):
            assert torch.equal(a, b)


def test_model_rejects_out_of_range_labels(device) -> None:
    """The target-range check enqueued at the start of the forward still raises
    at the loss (tensor_parallel/cross_entropy.py:109-114); ignored ids pass."""
    cfg = c1_config(layers=2)
    model = nm.GPTModel(cfg, activation_checkpoint_config=nm.ActivationCheckpointConfig(mode="full"))
    model = model.to(device=device, dtype=torch.bfloat16).train()
    ids = torch.randint(0, cfg.vocab_size, (2, 64), device=device)
    for bad in (cfg.vocab_size, -5):
        labels = ids.clone()
        labels[1, 7] = bad
        with pytest.raises(ValueError, match="outside the original"):
            model(ids, labels=labels)
    labels = ids.clone()
    labels[0, :5] = -100
    assert torch.isfinite(model(ids, labels=labels).loss)


def test_block_grads_accumulate_over_two_backward_passes(device) -> None:
    """The weight gradients (some computed on a second stream) are complete when
    the block's backward returns: a second pass accumulating into existing
    .grad tensors gives the bf16 sum of the two single-pass gradients."""
    x, w, meta = _block_inputs(device)
    dys = [torch.randn_like(x), torch.randn_like(x)]
    single = []
    for dy in dys:
        ws = [t.clone().requires_grad_(True) for t in w]
        B.CheckpointedBlockFunction.apply(x, meta, False, *ws).backward(dy)
        single.append([t.grad.clone() for t in ws])
    ws = [t.clone().requires_grad_(True) for t in w]
    for dy in dys:
        B.CheckpointedBlockFunction.apply(x, meta, False, *ws).backward(dy)
    for t, g1, g2 in zip(ws, *single):
        assert torch.equal(t.grad, g1 + g2)


def _block_saved_bytes(device, cfg, ids, ck) -> int:
    """Device memory one block leaves saved after the forward: a 2-layer minus a
    1-layer model's (embedding, final norm and LM-head state cancel)."""
    saved = []
    for layers in (1, 2):
        c = nm.GPTConfig(**{**cfg, "layers": layers})
        torch.manual_seed(0)
        model = nm.GPTModel(c, activation_checkpoint_config=ck).to(device=device, dtype=torch.bfloat16).train()
        model(ids, labels=ids)  # packs the block weights (new storage, old freed)
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        out = model(ids, labels=ids)
        torch.cuda.synchronize()
        saved.append(torch.cuda.memory_allocated() - base)
        out.loss.backward()
        del out, model
        torch.cuda.empty_cache()
    return saved[1] - saved[0]


def test_full_recompute_keeps_only_block_input(device) -> None:
    """A checkpointed block keeps exactly its bf16 input on the device; with
    offload_saved_tensors it keeps nothing there (the input waits in pinned host
    memory, the weights are never copied); without checkpointing it keeps every
    intermediate."""
    cfg = dict(hidden_size=512, ffn_hidden_size=1376, heads=8, seq_length=256, vocab_size=4096)
    ids = torch.randint(0, 4096, (4, 256), device=device)
    x_bytes = 4 * 256 * 512 * 2
    full = _block_saved_bytes(device, cfg, ids, nm.ActivationCheckpointConfig(mode="full"))
    off = _block_saved_bytes(device, cfg, ids, nm.ActivationCheckpointConfig(mode="full", offload_saved_tensors=True))
    none = _block_saved_bytes(device, cfg, ids, nm.ActivationCheckpointConfig(mode="none"))
    assert full == x_bytes, full
    assert off == 0, off
    assert none > 8 * x_bytes, none


@pytest.mark.parametrize("ops", [("attention", "mlp"), ("attention",), ("mlp",)])
def test_fused_selective_recompute_bit_identical_to_eager(device, ops) -> None:
    """Selective checkpointing on the fused block (models/gpt/layer.py:68-89):
    the chosen sub-blocks recomputed from their saved inputs with the
    forward's kernels, so the loss and every gradient equal the eager (no
    checkpoint) run's and the full-recompute run's bit for bit; offloading the
    sub-block inputs changes nothing either."""
    cfg = c1_config(layers=2, kv_heads=2)
    ids, labels = c1_batch()
    results = []
    for ck in (nm.ActivationCheckpointConfig(mode="none"), nm.ActivationCheckpointConfig(mode="full"),
               nm.ActivationCheckpointConfig(mode="selective", selective_ops=ops),
               nm.ActivationCheckpointConfig(mode="selective", selective_ops=ops, offload_saved_tensors=True)):
        torch.manual_seed(0)
        model = nm.GPTModel(cfg, activation_checkpoint_config=ck).to(device=device, dtype=torch.bfloat16).train()
        assert all(layer.fusable() for layer in model.layers)
        loss = model(ids.to(device), labels=labels.to(device)).loss
        loss.backward()
        results.append((loss.detach(), [p.grad.clone() for p in model.parameters()]))
    for loss, grads in results[1:]:
        assert torch.equal(loss, results[0][0])
        for a, b in zip(grads, results[0][1]):
            assert torch.equal(a, b)


def test_fused_selective_keeps_the_sub_block_inputs(device) -> None:
    """Selective recompute of both sub-blocks keeps what the reference's
    checkpoint boundaries keep: the block input, the residual midpoint and the
    two checkpointed sub-blocks' inputs (4 x the input's bytes); with
    offload_saved_tensors the sub-block inputs wait in host memory (2 x);
    checkpointing only the MLP keeps the attention's intermediates too."""
    cfg = dict(hidden_size=512, ffn_hidden_size=1376, heads=8, seq_length=256, vocab_size=4096)
    ids = torch.randint(0, 4096, (4, 256), device=device)
    x_bytes = 4 * 256 * 512 * 2
    sel = _block_saved_bytes(device, cfg, ids, nm.ActivationCheckpointConfig(mode="selective"))
    off = _block_saved_bytes(device, cfg, ids, nm.ActivationCheckpointConfig(mode="selective",
                                                                              offload_saved_tensors=True))
    mlp = _block_saved_bytes(device, cfg, ids, nm.ActivationCheckpointConfig(mode="selective",
                                                                              selective_ops=("mlp",)))
    assert sel == 4 * x_bytes, sel
    assert off == 2 * x_bytes, off
    assert mlp > 6 * x_bytes, mlp


def test_offload_and_block_interval_match_oracle_and_full_recompute(device) -> None:
    """offload_saved_tensors=True and block_interval=2 (layers 0 and 2
    checkpointed, 1 and 3 eager; models/gpt/model.py:162-170) give the loss and
    gradients of plain full recompute bit for bit, and match the oracle run with
    the same switch (bf16 tolerance)."""
    cfg = c1_config(layers=4, kv_heads=2)
    ids, labels = c1_batch()
    results = {}
    for name, ck in (("full", nm.ActivationCheckpointConfig(mode="full")),
                     ("offload", nm.ActivationCheckpointConfig(mode="full", offload_saved_tensors=True)),
                     ("interval2", nm.ActivationCheckpointConfig(mode="full", block_interval=2))):
        torch.manual_seed(0)
        ours = nm.GPTModel(cfg, activation_checkpoint_config=ck).to(device=device, dtype=torch.bfloat16).train()
        lo = ours(ids.to(device), labels=labels.to(device)).loss
        lo.backward()
        results[name] = (lo.detach(), {n: p.grad.clone() for n, p in ours.named_parameters()})
        if name == "interval2":
            state = {k: v.cpu() for k, v in ours.state_dict().items()}
            torch.manual_seed(0)
            ref = R.OracleGPTModel(cfg, activation_checkpoint_config=ck).to(dtype=torch.bfloat16).train()
            ref.load_state_dict(state)
            ref32 = R.OracleGPTModel(cfg, activation_checkpoint_config=ck).train()
            ref32.load_state_dict({k: v.float() for k, v in state.items()})
            lr = ref(ids, labels=labels).loss
            lr.backward()
            ref32(ids, labels=labels).loss.backward()
            assert_loss_close(lo, lr, torch.bfloat16)
            assert_bf16_grads(ours, ref, ref32)
            assert [layer.forward_calls for layer in ref.layers] == [2, 1, 2, 1]
    base_loss, base_grads = results["full"]
    for name in ("offload", "interval2"):
        loss, grads = results[name]
        assert torch.equal(loss, base_loss), name
        for n, g in grads.items():
            assert torch.equal(g, base_grads[n]), (name, n)


def test_explicit_position_ids_match_oracle(device) -> None:
    """position_ids given as [B, S] ids (not a range): RoPE at those positions and
    the causal mask's query offset position_ids[0] (models/gpt/model.py:193-200,
    attention.py:180-206), against the oracle; a range given as 1-D ids takes the
    offset form and equals the default; negative ids raise."""
    cfg = c1_config(layers=2, kv_heads=2)
    ours, ref, ref32 = build_pair(cfg, "full", torch.bfloat16, device)
    ids, labels = c1_batch()
    g = torch.Generator().manual_seed(4)
    pos = torch.stack([torch.randperm(600, generator=g)[:128] for _ in range(4)])
    pos[0, 0] = 3
    check_model(ours, ref, ref32, torch.bfloat16, ids, labels, device, position_ids=pos)
    with torch.no_grad():
        a = ours(ids.to(device), labels=labels.to(device)).loss
        b = ours(ids.to(device), labels=labels.to(device), position_ids=torch.arange(128, device=device)).loss
        assert torch.equal(a, b)
        with pytest.raises(ValueError, match="non-negative"):
            ours(ids.to(device), labels=labels.to(device), position_ids=pos.to(device) - 5)


def test_c4_width_block_matches_oracle_layer(device) -> None:
    """One config-4 block (hidden 2048, 32 query / 8 KV heads of 64, SwiGLU 5632)
    at B1 S2048 in bf16, checkpointed, against the oracle's GPTLayer: the output,
    a loss made of it and every gradient (input and the nine weights)."""
    cfg = nm.GPTConfig(layers=1, hidden_size=2048, ffn_hidden_size=5632, heads=32, kv_heads=8,
                       seq_length=2048, vocab_size=8192, norm_epsilon=1e-5, rope_theta=1e4)
    torch.manual_seed(0)
    layer = R.OracleLayer(cfg, 0, dtype=torch.bfloat16)
    with torch.no_grad():  # norms away from 1 so their gradients are exercised
        layer.input_norm.weight.add_(0.1 * torch.randn(2048).bfloat16())
        layer.post_attention_norm.weight.add_(0.1 * torch.randn(2048).bfloat16())
    layer32 = R.OracleLayer(cfg, 0)
    layer32.load_state_dict({k: v.float() for k, v in layer.state_dict().items()})
    g = torch.Generator().manual_seed(6)
    x = torch.randn(1, 2048, 2048, generator=g).bfloat16()
    dy = torch.randn(1, 2048, 2048, generator=g).bfloat16()
    xr = x.clone().requires_grad_(True)
    yr = layer(xr, position_ids=torch.arange(2048), sequence_offset=0)
    loss_r = (yr.float() * dy.float()).sum()
    loss_r.backward()
    x32 = x.float().requires_grad_(True)
    (layer32(x32, position_ids=torch.arange(2048), sequence_offset=0) * dy.float()).sum().backward()
    params32 = dict(layer32.named_parameters())
    names = ("input_norm.weight", "attention.q_proj.linear.weight", "attention.k_proj.linear.weight",
             "attention.v_proj.linear.weight", "attention.out_proj.linear.weight",
             "post_attention_norm.weight", "mlp.gate_proj.linear.weight", "mlp.up_proj.linear.weight",
             "mlp.down_proj.linear.weight")
    params = dict(layer.named_parameters())
    ws = [params[n].detach().to(device).requires_grad_(True) for n in names]
    tab = nm.RotaryEmbedding(64).tables(device, 2048)
    meta = B.BlockMeta(heads=32, kv_heads=8, head_dim=64, eps=1e-5, sequence_offset=0, cos=tab.cos,
                       sin=tab.sin, positions=None)
    xd = x.to(device).requires_grad_(True)
    yd = B.CheckpointedBlockFunction.apply(xd, meta, False, *ws)
    loss_d = (yd.float() * dy.to(device).float()).sum()
    loss_d.backward()
    assert_close_scaled(yd, yr, torch.bfloat16, msg="y")
    assert_loss_close(loss_d, loss_r, torch.bfloat16, msg="sum(y * dy)")
    assert_bf16_grad(xd.grad, xr.grad, x32.grad, msg="x")
    for n, w in zip(names, ws):
        assert_bf16_grad(w.grad, params[n].grad, params32[n].grad, msg=n)


def test_c3_model_step_full_and_none_bit_identical(device) -> None:
    """The 24-layer config-3 model (310.8M parameters, B16 S512, bf16) with full
    recompute and without checkpointing: the same loss and every gradient bit
    for bit, all finite."""
    cfg = nm.GPTConfig(layers=24, hidden_size=1024, ffn_hidden_size=2736, heads=16, seq_length=512,
                       vocab_size=8192, norm_epsilon=1e-5, rope_theta=1e4)
    g = torch.Generator(device=device).manual_seed(1234)
    ids = torch.randint(0, 8192, (16, 513), device=device, generator=g)
    x, y = ids[:, :512].contiguous(), ids[:, 1:].contiguous()
    results = []
    for mode in ("full", "none"):
        torch.manual_seed(1234)
        model = nm.GPTModel(cfg, activation_checkpoint_config=nm.ActivationCheckpointConfig(mode=mode))
        model = model.to(device=device, dtype=torch.bfloat16).train()
        loss = model(x, labels=y).loss
        loss.backward()
        results.append((loss.detach(), [p.grad for p in model.parameters()]))
        del model
    (l0, g0), (l1, g1) = results
    assert torch.isfinite(l0) and torch.equal(l0, l1)
    assert len(g0) == len(g1) == 24 * 9 + 2
    for a, b in zip(g0, g1):
        assert bool(torch.isfinite(a).all()) and torch.equal(a, b)


def _deep_model_matches_oracle(device, cfg, batch, seq) -> None:
    """The whole model at depth, bf16 with full recompute on the GPU, against
    the oracle in bf16 and in fp32 (no checkpointing there: its gradients
    equal the checkpointed ones, pinned in tests/test_oracle.py), seeded
    uniform tokens: the loss and every gradient."""
    ck = nm.ActivationCheckpointConfig(mode="full")
    torch.manual_seed(1234)
    ours = nm.GPTModel(cfg, activation_checkpoint_config=ck).to(device=device, dtype=torch.bfloat16).train()
    state = {k: v.cpu() for k, v in ours.state_dict().items()}
    g = torch.Generator().manual_seed(1234)
    ids = torch.randint(0, cfg.vocab_size, (batch, seq + 1), generator=g)
    x, y = ids[:, :seq].contiguous(), ids[:, 1:].contiguous()
    lo = ours(x.to(device), labels=y.to(device)).loss
    lo.backward()
    torch.cuda.synchronize()
    none = nm.ActivationCheckpointConfig(mode="none")
    ref = R.OracleGPTModel(cfg, activation_checkpoint_config=none).to(dtype=torch.bfloat16).train()
    ref.load_state_dict(state)
    lr = ref(x, labels=y).loss
    lr.backward()
    ref32 = R.OracleGPTModel(cfg, activation_checkpoint_config=none).train()
    ref32.load_state_dict({k: v.float() for k, v in state.items()})
    ref32(x, labels=y).loss.backward()
    assert_loss_close(lo, lr, torch.bfloat16)
    assert_bf16_grads(ours, ref, ref32)


@pytest.mark.timeout(900)
def test_c3_model_matches_oracle(device) -> None:
    """Config 3's 24-layer, 310.8M-parameter model at one 512-token sequence."""
    cfg = nm.GPTConfig(layers=24, hidden_size=1024, ffn_hidden_size=2736, heads=16, seq_length=512,
                       vocab_size=8192, norm_epsilon=1e-5, rope_theta=1e4)
    _deep_model_matches_oracle(device, cfg, 1, 512)


@pytest.mark.timeout(900)
def test_c4_model_matches_oracle(device) -> None:
    """Config 4's 16-layer GQA model (hidden 2048, 32 query / 8 KV heads,
    SwiGLU 5632, 738.3M parameters) at one 2048-token sequence."""
    cfg = nm.GPTConfig(layers=16, hidden_size=2048, ffn_hidden_size=5632, heads=32, kv_heads=8,
                       seq_length=2048, vocab_size=8192, norm_epsilon=1e-5, rope_theta=1e4)
    _deep_model_matches_oracle(device, cfg, 1, 2048)


@pytest.mark.parametrize("dtype,bias,tie,mode", [
    (torch.float32, True, True, "full"), (torch.float32, False, False, "full"),
    (torch.bfloat16, True, False, "none"), (torch.bfloat16, False, False, "full"),
])
def test_bias_and_untied_head_match_oracle(device, dtype, bias, tie, mode) -> None:
    """GPTConfig.bias (column biases in the nn.Linear, row biases added after
    the product; tensor_parallel/layers.py:27-155) and tie_embeddings=False
    (the LM head's own N(0, 0.02) weight; models/gpt/model.py:125-142): loss and
    every gradient against the oracle (fp32 rtol 1e-5; bf16 2e-2 / 1e-2).
    Layers with biases run the module path; an untied head keeps the fused one."""
    cfg = c1_config(layers=2, bias=bias, tie_embeddings=tie)
    ours, ref, ref32 = build_pair(cfg, mode, dtype, device)
    assert (ours.lm_head.weight is ours.embedding.weight) == tie
    ids, labels = c1_batch()
    check_model(ours, ref, ref32, dtype, ids, labels, device)


@pytest.mark.parametrize("dtype,tie", [(torch.float32, True), (torch.bfloat16, True), (torch.bfloat16, False)])
def test_vocabulary_not_a_multiple_of_8_matches_oracle(device, dtype, tie) -> None:
    """A 1001-token vocabulary (the reference takes any size; the kernels move
    16-byte chunks, so the LM head runs on a zero-padded table with -inf logits
    in the padding): loss and every gradient, and the logits of the
    label-free forward, against the oracle."""
    cfg = c1_config(layers=2, vocab_size=1001, tie_embeddings=tie)
    ours, ref, ref32 = build_pair(cfg, "full", dtype, device)
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, 1001, (2, 129), generator=g)
    x, y = ids[:, :128].contiguous(), ids[:, 1:].contiguous()
    y[0, :3] = -100
    y[1, 5] = 1000  # the last real token
    check_model(ours, ref, ref32, dtype, x, y, device)
    with torch.no_grad():
        logits = ours(x.to(device)).logits
        rlog = ref(x).logits
    assert logits.shape == (2, 128, 1001)
    assert_close_scaled(logits, rlog, dtype, msg="logits")


def test_head_size_96_model_matches_oracle(device) -> None:
    """hidden 384 over 4 heads (head size 96) in bf16: the layers leave the
    fused block (its attention kernels take 64 and 128) for the module path;
    loss and every gradient against the oracle."""
    cfg = c1_config(layers=2, hidden_size=384, ffn_hidden_size=1024, heads=4, kv_heads=2)
    ours, ref, ref32 = build_pair(cfg, "full", torch.bfloat16, device)
    assert not any(layer.fusable() for layer in ours.layers)
    ids, labels = c1_batch()
    check_model(ours, ref, ref32, torch.bfloat16, ids, labels, device)


def test_pipeline_stage_split_equals_the_whole_model(device) -> None:
    """Two stages of one model (models/gpt/model.py:40-250 with layer_start /
    layer_end and the owns_* flags, chained through hidden_states as a
    pipeline does at one rank): the loss and every gradient equal the whole
    model's, bit for bit."""
    cfg = c1_config(layers=4, tie_embeddings=False)
    torch.manual_seed(0)
    whole = nm.GPTModel(cfg).to(device=device, dtype=torch.bfloat16).train()
    first = nm.GPTModel(cfg, layer_end=2, owns_lm_head=False, owns_final_norm=False)
    last = nm.GPTModel(cfg, layer_start=2, owns_embedding=False)
    first = first.to(device=device, dtype=torch.bfloat16).train()
    last = last.to(device=device, dtype=torch.bfloat16).train()
    state = whole.state_dict()
    first.load_state_dict({k: v for k, v in state.items()
                           if k.startswith("embedding.") or k.split(".")[:2] in (["layers", "0"], ["layers", "1"])})
    moved = {}
    for k, v in state.items():
        parts = k.split(".")
        if parts[0] == "layers" and int(parts[1]) >= 2:
            moved[".".join(["layers", str(int(parts[1]) - 2), *parts[2:]])] = v
        elif parts[0] in ("final_norm", "lm_head"):
            moved[k] = v
    last.load_state_dict(moved)
    ids, labels = c1_batch()
    ids, labels = ids[:2].to(device), labels[:2].to(device)
    loss = whole(ids, labels=labels).loss
    loss.backward()
    hidden = first(ids).hidden_states
    assert first.lm_head is None and last.embedding is None
    staged = last(hidden_states=hidden, labels=labels).loss
    staged.backward()
    assert torch.equal(loss, staged)
    grads = dict(whole.named_parameters())
    for name, p in first.named_parameters():
        assert torch.equal(p.grad, grads[name].grad), name
    for name, p in last.named_parameters():
        parts = name.split(".")
        src = ".".join(["layers", str(int(parts[1]) + 2), *parts[2:]]) if parts[0] == "layers" else name
        assert torch.equal(p.grad, grads[src].grad), name


def test_activation_checkpoint_module_wrapper(device) -> None:
    """nn/activation_checkpoint.py:103-131: the module wrapper runs the wrapped
    layer under the checkpoint; output and gradients equal the unwrapped
    layer's bit for bit."""
    cfg = c1_config(layers=1)
    torch.manual_seed(0)
    model = nm.GPTModel(cfg).to(device=device, dtype=torch.bfloat16)
    layer = model.layers[0]
    x = torch.randn(2, 64, cfg.hidden_size, device=device).bfloat16()
    calls = []
    hook = layer.register_forward_hook(lambda *a: calls.append(1))
    outs, grads = [], []
    for wrapped in (False, True):
        layer.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_(True)
        mod = nm.ActivationCheckpoint(layer) if wrapped else layer
        y = mod(xi)
        y.float().square().sum().backward()
        outs.append(y.detach())
        grads.append([xi.grad] + [p.grad.clone() for p in layer.parameters()])
    hook.remove()
    assert len(calls) >= 2
    assert torch.equal(outs[0], outs[1])
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_precision_modes_run_or_raise(device) -> None:
    """The reference's precision modes (config/schema.py:55-64,
    training/trainer.py:49-57): bf16 parameters under torch.autocast to
    bfloat16 (the configurations' mode, as the reference's trainer wraps it)
    run and equal the same step without autocast bit for bit; float32
    parameters under autocast to bfloat16 (params=float32/compute=bfloat16)
    and float16 parameters raise a ValueError naming the mode, at the model,
    at the kernel seam's modules and at the functional entry points."""
    cfg = c1_config(layers=2, kv_heads=2)
    ids, labels = c1_batch()
    ids, labels = ids.to(device), labels.to(device)
    torch.manual_seed(0)
    model = nm.GPTModel(cfg).to(device=device, dtype=torch.bfloat16).train()
    plain = model(ids, labels=labels).loss
    with torch.autocast("cuda", dtype=torch.bfloat16):
        cast = model(ids, labels=labels).loss
    assert torch.equal(plain, cast)
    model32 = nm.GPTModel(cfg).to(device=device).train()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        with pytest.raises(ValueError, match="params=float32/compute=bfloat16"):
            model32(ids, labels=labels)
        lin = nm.HipKernelBackend().linear(256, 64, bias=False, device=device)
        with pytest.raises(ValueError, match="params=float32/compute=bfloat16"):
            lin(torch.randn(8, 256, device=device))
        q = torch.randn(1, 4, 64, 64, device=device)
        with pytest.raises(ValueError, match="params=float32/compute=bfloat16"):
            nm.HipKernelBackend().local_attention(q, q, q)
        with pytest.raises(ValueError, match="params=float32/compute=bfloat16"):
            nm.rms_norm(q, torch.ones(64, device=device), 1e-5)
    model16 = nm.GPTModel(cfg).to(device=device, dtype=torch.float16).train()
    with pytest.raises(ValueError, match="float16.*supported"):
        model16(ids, labels=labels)
    with pytest.raises(ValueError, match="float16.*supported"):
        nm.attention(q.half(), q.half(), q.half())
