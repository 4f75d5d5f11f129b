"""Pin the CPU oracle against independent definitions (no GPU).

Each oracle function is checked against something other than its own
formula: a PyTorch library routine implementing the same textbook op
(F.rms_norm, F.scaled_dot_product_attention, F.cross_entropy,
torch.optim.AdamW), a closed-form derivative, an fp64 brute-force loop on tiny
inputs, or an invariant.  Mirrors the reference's own hot-path tests
(tests/unit/test_gpt_kernels.py:16-78, test_tensor_parallel_layers.py:108-166,
test_context_parallel.py:29-124, test_gpt_model.py:69-88, 245-309).
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import reference as R


# ---------------------------------------------------------------- RMSNorm
def test_rms_norm_matches_closed_form_fp64() -> None:
    """tests/unit/test_gpt_kernels.py:16-21 of the reference."""
    torch.manual_seed(11)
    x = torch.randn(2, 3, 8, dtype=torch.float64)
    w = torch.ones(8, dtype=torch.float64)
    expected = x * torch.rsqrt(x.square().mean(dim=-1, keepdim=True) + 1.0e-5)
    torch.testing.assert_close(R.rms_norm(x, w, 1.0e-5), expected, rtol=1e-6, atol=1e-6)


def test_rms_norm_matches_torch_rms_norm() -> None:
    torch.manual_seed(0)
    x = torch.randn(5, 33, dtype=torch.float64)
    w = torch.randn(33, dtype=torch.float64)
    # nn/norms.py:39-40 takes the statistics through x.float(), i.e. fp32 even for
    # fp64 input, hence the fp32-level tolerance
    torch.testing.assert_close(R.rms_norm(x, w, 1e-5), F.rms_norm(x, (33,), w, 1e-5),
                               rtol=1e-6, atol=1e-6)


def test_rms_norm_bf16_rounds_before_weight() -> None:
    """nn/norms.py:41: cast(n) * cast(w) -- rounding n first differs from rounding n*w once."""
    torch.manual_seed(1)
    x = torch.randn(64, 128).bfloat16()
    w = (torch.rand(128) + 0.5).bfloat16()
    y = R.rms_norm(x, w, 1e-5)
    n = x.float() * torch.rsqrt(x.float().square().mean(-1, keepdim=True) + 1e-5)
    two_step = (n.bfloat16().float() * w.float()).bfloat16()
    assert torch.equal(y, two_step)


def test_rms_norm_backward_closed_form() -> None:
    """dx = rstd (g - n mean(g n)), dw = sum dy n, g = dy w."""
    torch.manual_seed(2)
    x = torch.randn(6, 17, dtype=torch.float64, requires_grad=True)
    w = torch.randn(17, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(6, 17, dtype=torch.float64)
    R.rms_norm(x, w, 1e-5).backward(dy)
    r = torch.rsqrt(x.detach().square().mean(-1, keepdim=True) + 1e-5)
    n = x.detach() * r
    g = dy * w.detach()
    dx = r * (g - n * (g * n).mean(-1, keepdim=True))
    torch.testing.assert_close(x.grad, dx, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(w.grad, (dy * n).sum(0), rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- RoPE
def test_rope_preserves_norms() -> None:
    """tests/unit/test_gpt_kernels.py:24-32 of the reference."""
    cos, sin = R.rope_cos_sin(torch.arange(6), 8, 1e4, torch.float32)
    q = torch.randn(2, 4, 6, 8)
    k = torch.randn(2, 2, 6, 8)
    rq, rk = R.apply_rotary_pos_emb(q, k, cos, sin)
    torch.testing.assert_close(rq.norm(dim=-1), q.norm(dim=-1))
    torch.testing.assert_close(rk.norm(dim=-1), k.norm(dim=-1))


def test_rope_matches_complex_rotation_bruteforce() -> None:
    """NeoX halves: the pair (x_i, x_{i+D/2}) is the complex number rotated by p * inv_freq_i."""
    d, s = 16, 9
    theta = 1e4
    q = torch.randn(1, 2, s, d, dtype=torch.float64)
    cos, sin = R.rope_cos_sin(torch.arange(s), d, theta, torch.float64)
    rq, _ = R.apply_rotary_pos_emb(q, q, cos, sin)
    out = torch.empty_like(q)
    for p in range(s):
        for i in range(d // 2):
            ang = p * (1.0 / theta ** (2 * i / d))
            z = complex(q[0, 0, p, i].item(), q[0, 0, p, i + d // 2].item()) * complex(math.cos(ang), math.sin(ang))
            out[0, 0, p, i], out[0, 0, p, i + d // 2] = z.real, z.imag
    torch.testing.assert_close(rq[0, 0], out[0, 0], rtol=1e-6, atol=1e-6)


def test_rope_position_zero_is_identity_and_negative_sin_inverts() -> None:
    d = 8
    cos, sin = R.rope_cos_sin(torch.arange(5), d, 1e4, torch.float64)
    q = torch.randn(1, 1, 5, d, dtype=torch.float64)
    rq, _ = R.apply_rotary_pos_emb(q, q, cos, sin)
    torch.testing.assert_close(rq[:, :, 0], q[:, :, 0])
    back, _ = R.apply_rotary_pos_emb(rq, rq, cos, -sin)
    torch.testing.assert_close(back, q)


# ---------------------------------------------------------------- attention
def _brute_attention(q, k, v, causal, q_off=0, k_off=0, mask=None):
    """Softmax attention by loops.  mask (broadcast to [b, h, sq, sk]): a
    boolean mask drops the False keys, a floating one is added to the scores;
    a row with no visible key gives zeros."""
    b, h, sq, d = q.shape
    rep = h // k.shape[1]
    out = torch.zeros_like(q)
    if mask is not None:
        mask = torch.broadcast_to(mask, (b, h, sq, k.shape[2]))
    for bi in range(b):
        for hi in range(h):
            kh = hi // rep
            for i in range(sq):
                scores = []
                for j in range(k.shape[2]):
                    visible = not (causal and k_off + j > q_off + i)
                    extra = 0.0
                    if mask is not None:
                        if mask.dtype == torch.bool:
                            visible = visible and bool(mask[bi, hi, i, j])
                        else:
                            extra = float(mask[bi, hi, i, j])
                    if visible:
                        scores.append(float(q[bi, hi, i] @ k[bi, kh, j]) / math.sqrt(d) + extra)
                    else:
                        scores.append(-math.inf)
                m = max(scores)
                if m == -math.inf:
                    continue
                w = [math.exp(s - m) for s in scores]
                tot = sum(w)
                out[bi, hi, i] = sum(wj / tot * v[bi, kh, j] for j, wj in enumerate(w))
    return out


@pytest.mark.parametrize("causal,offset", [(True, 0), (True, 3), (False, 0)])
def test_local_attention_matches_bruteforce(causal, offset) -> None:
    torch.manual_seed(3)
    q = torch.randn(1, 4, 5, 8, dtype=torch.float64)
    k = torch.randn(1, 2, 7, 8, dtype=torch.float64)
    v = torch.randn(1, 2, 7, 8, dtype=torch.float64)
    if causal and offset == 0:
        k, v = k[:, :, :5], v[:, :, :5]
    got = R.local_attention(q, k, v, causal=causal, sequence_offset=offset)
    torch.testing.assert_close(got, _brute_attention(q, k, v, causal, q_off=offset))


@pytest.mark.parametrize("causal,offset,kind", [(True, 0, "bool"), (True, 2, "bool"), (False, 0, "bool"),
                                                (False, 0, "add")])
def test_local_attention_with_mask_matches_bruteforce(causal, offset, kind) -> None:
    """attention_mask as torch_backend.py:60-66 combines it: ANDed with the
    causal mask (a boolean mask), or added to the scores (a floating mask,
    without causal); a query row whose keys are all masked gives zeros (the
    CPU SDPA's safe softmax), checked by loops."""
    torch.manual_seed(5)
    q = torch.randn(2, 4, 5, 8, dtype=torch.float64)
    k = torch.randn(2, 2, 7, 8, dtype=torch.float64)
    v = torch.randn(2, 2, 7, 8, dtype=torch.float64)
    if kind == "bool":
        mask = torch.rand(2, 1, 5, 7) > 0.3
        mask[1, 0, 2] = False  # a fully masked row
    else:
        mask = torch.randn(5, 7, dtype=torch.float64)
        mask[3, 1:5] = -math.inf
    got = R.local_attention(q, k, v, causal=causal, sequence_offset=offset, attention_mask=mask)
    torch.testing.assert_close(got, _brute_attention(q, k, v, causal, q_off=offset, mask=mask))


def test_local_attention_is_causal_and_gqa_is_repeat() -> None:
    """tests/unit/test_gpt_kernels.py:35-59 of the reference."""
    torch.manual_seed(3)
    q, k, v = (torch.randn(1, 2, 4, 8) for _ in range(3))
    changed = v.clone()
    changed[..., 1:, :] += 100.0
    torch.testing.assert_close(R.local_attention(q, k, v)[..., 0, :], R.local_attention(q, k, changed)[..., 0, :])
    q = torch.randn(1, 4, 3, 8)
    k = torch.randn(1, 2, 3, 8)
    v = torch.randn(1, 2, 3, 8)
    torch.testing.assert_close(
        R.local_attention(q, k, v),
        R.local_attention(q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1)),
    )


def test_ring_equals_full_attention_over_concatenated_blocks() -> None:
    """Ring maths == all-gather attention with absolute offsets (context_parallel/all_gather.py:81-113)."""
    torch.manual_seed(4)
    sq, nb = 6, 3
    q = torch.randn(1, 4, sq, 8, dtype=torch.float64, requires_grad=True)
    blocks = [(torch.randn(1, 2, sq, 8, dtype=torch.float64, requires_grad=True),
               torch.randn(1, 2, sq, 8, dtype=torch.float64, requires_grad=True)) for _ in range(nb)]
    rank = 2
    offsets = [r * sq for r in (2, 1, 0)]  # ring order (rank - step) % size
    order = [blocks[r] for r in (2, 1, 0)]
    out, lse = R.ring_attention_forward(q, order, offsets, causal=True, query_offset=rank * sq)
    kc = torch.cat([b[0] for b in blocks], dim=2)
    vc = torch.cat([b[1] for b in blocks], dim=2)
    full = R.local_attention(q, kc, vc, causal=True, sequence_offset=rank * sq)
    torch.testing.assert_close(out, full)
    # lse == logsumexp of the masked scores
    scores = (q @ kc.repeat_interleave(2, 1).transpose(-1, -2)) / math.sqrt(8)
    mask = torch.arange(nb * sq)[None, :] <= (rank * sq + torch.arange(sq))[:, None]
    ref_lse = scores.masked_fill(~mask, -math.inf).logsumexp(-1, keepdim=True)
    torch.testing.assert_close(lse, ref_lse)
    # backward == autograd of the full attention
    go = torch.randn_like(out)
    dq, dks, dvs = R.ring_attention_backward(go, q.detach(), [(k.detach(), v.detach()) for k, v in order],
                                             offsets, out.detach(), lse, causal=True, query_offset=rank * sq)
    full.backward(go)
    torch.testing.assert_close(dq, q.grad)
    for (k, v), dk, dv in zip(order, dks, dvs):
        torch.testing.assert_close(dk, k.grad)
        torch.testing.assert_close(dv, v.grad)


# ---------------------------------------------------------------- SwiGLU
def test_swiglu_closed_form_gradient() -> None:
    g = torch.randn(40, dtype=torch.float64, requires_grad=True)
    u = torch.randn(40, dtype=torch.float64, requires_grad=True)
    dh = torch.randn(40, dtype=torch.float64)
    R.swiglu(g, u).backward(dh)
    sig = torch.sigmoid(g.detach())
    torch.testing.assert_close(g.grad, dh * u.detach() * sig * (1 + g.detach() * (1 - sig)))
    torch.testing.assert_close(u.grad, dh * g.detach() * sig)


# ---------------------------------------------------------------- cross entropy
@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
def test_cross_entropy_matches_torch(reduction: str) -> None:
    """tests/unit/test_tensor_parallel_layers.py:108-136 of the reference."""
    torch.manual_seed(7)
    logits = torch.randn(2, 3, 7, dtype=torch.float64, requires_grad=True)
    ref = logits.detach().clone().requires_grad_(True)
    targets = torch.tensor([[0, 3, 6], [2, -100, 1]])
    got = R.cross_entropy_tokens(logits, targets, reduction=reduction)
    exp = F.cross_entropy(ref.reshape(-1, 7), targets.reshape(-1), reduction=reduction, ignore_index=-100)
    if reduction == "none":
        exp = exp.view_as(targets)
        grad = torch.randn_like(got)
        got.backward(grad)
        exp.backward(grad)
    else:
        got.backward()
        exp.backward()
    torch.testing.assert_close(got, exp)
    torch.testing.assert_close(logits.grad, ref.grad)


def test_cross_entropy_bf16_uses_fp32_and_rejects_bad_targets() -> None:
    """tests/unit/test_tensor_parallel_layers.py:139-170 of the reference."""
    logits = torch.zeros(1, 70_000, dtype=torch.bfloat16, requires_grad=True)
    ref = logits.detach().float().requires_grad_(True)
    t = torch.tensor([0])
    got = R.cross_entropy_tokens(logits, t, reduction="mean")
    exp = F.cross_entropy(ref, t)
    got.backward()
    exp.backward()
    assert got.dtype is torch.float32
    torch.testing.assert_close(got, exp)
    assert logits.grad.dtype is torch.bfloat16
    torch.testing.assert_close(logits.grad.float(), ref.grad, rtol=5e-3, atol=1e-7)
    with pytest.raises(ValueError):
        R.cross_entropy_tokens(torch.zeros(1, 4), torch.tensor([4]))


# ---------------------------------------------------------------- AdamW
def test_adamw_master_step_matches_torch_adamw() -> None:
    torch.manual_seed(5)
    p0 = torch.randn(100)
    ref = p0.clone().requires_grad_(True)
    opt = torch.optim.AdamW([ref], lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    master, m, v = p0.clone(), torch.zeros(100), torch.zeros(100)
    for step in range(1, 6):
        g = torch.randn(100)
        ref.grad = g.clone()
        opt.step()
        oracle.adamw_master_step(master, m, v, g, step=step, lr=3e-4, weight_decay=0.1)
    torch.testing.assert_close(master, ref.detach(), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("scale,max_norm", [(3.0, 1.0), (1e-2, 1.0), (1e-7, 1e-6), (0.0, 1.0)])
def test_clip_coefficient_matches_torch_clip_grad_norm(scale, max_norm) -> None:
    """The factor ``torch.nn.utils.clip_grad_norm_`` multiplies the gradients by
    (max_norm / (norm + 1e-6), clamped at 1) equals the oracle's coefficient
    (data_parallel/_zero.py:160-163).  The 1e-7 case makes the 1e-6 term decide
    the result (dropping it or moving it would change the coefficient by ~2x);
    the 1e-2 and 0 cases sit under the clamp."""
    g = torch.Generator().manual_seed(17)
    grads = [torch.randn(*s, generator=g, dtype=torch.float64) * scale for s in ((7, 5), (11,), (3, 2, 4))]
    params = [torch.nn.Parameter(torch.zeros_like(t)) for t in grads]
    for p, t in zip(params, grads):
        p.grad = t.clone()
    norm = torch.nn.utils.clip_grad_norm_(params, max_norm)
    coef = R.clip_coefficient(norm, max_norm)
    for p, t in zip(params, grads):
        torch.testing.assert_close(p.grad, t * coef, rtol=1e-12, atol=0)
    if scale == 3.0:
        assert coef < 0.2
    if scale <= 1e-2 and scale != 1e-7:
        assert coef == 1.0
    if scale == 1e-7:
        expected_no_eps = max_norm / float(norm)
        assert abs(float(coef) - expected_no_eps) > 0.05 * expected_no_eps


def test_clip_then_adamw_master_step_matches_torch() -> None:
    """One ZeRO optimizer step at DP=1 (_zero.py:130-199): the global-norm clip
    followed by the fp32-master AdamW, against clip_grad_norm_ + torch AdamW."""
    g = torch.Generator().manual_seed(23)
    shapes = ((40,), (6, 9))
    init = [torch.randn(*s, generator=g) for s in shapes]
    params = [torch.nn.Parameter(t.clone()) for t in init]
    opt = torch.optim.AdamW(params, lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    master = [t.clone() for t in init]
    m = [torch.zeros_like(t) for t in init]
    v = [torch.zeros_like(t) for t in init]
    for step in range(1, 4):
        grads = [torch.randn(*s, generator=g) * 2.0 for s in shapes]
        for p, t in zip(params, grads):
            p.grad = t.clone()
        torch.nn.utils.clip_grad_norm_(params, 1.0)
        opt.step()
        norm = torch.sqrt(sum((t * t).sum() for t in grads))
        coef = R.clip_coefficient(norm, 1.0)
        for w, mm, vv, t in zip(master, m, v, grads):
            R.adamw_master_step(w, mm, vv, t * coef, step=step, lr=1e-2, weight_decay=0.1)
    for p, w in zip(params, master):
        torch.testing.assert_close(w, p.detach(), rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- embedding
def test_embedding_lookup_masks_ids_outside_the_table() -> None:
    """VocabParallelEmbedding at TP=1 (tensor_parallel/embedding.py:63-68): ids in
    [0, V) gather their row, ids outside give zero rows and pass no gradient;
    checked against an explicit per-token loop and an index_add of the in-range
    rows only."""
    g = torch.Generator().manual_seed(3)
    vocab, hidden = 10, 4
    w = torch.randn(vocab, hidden, generator=g, dtype=torch.float64, requires_grad=True)
    ids = torch.tensor([[0, 9, -1, 10, 3], [3, -100, 7, 25, 0]])
    out = R.embedding_lookup(ids, w)
    for b in range(ids.shape[0]):
        for t in range(ids.shape[1]):
            i = int(ids[b, t])
            exp = w[i] if 0 <= i < vocab else torch.zeros(hidden, dtype=torch.float64)
            assert torch.equal(out[b, t], exp)
    dout = torch.randn(*ids.shape, hidden, generator=g, dtype=torch.float64)
    out.backward(dout)
    inside = (ids >= 0) & (ids < vocab)
    exp_grad = torch.zeros(vocab, hidden, dtype=torch.float64).index_add_(
        0, ids[inside], dout[inside])
    torch.testing.assert_close(w.grad, exp_grad, rtol=0, atol=1e-15)
    with pytest.raises(TypeError):
        R.embedding_lookup(ids.float(), w)


# ---------------------------------------------------------------- model
class _Cfg:
    layers = 2
    hidden_size = 32
    ffn_hidden_size = 48
    heads = 4
    kv_heads = 2
    vocab_size = 64
    rope_theta = 1e4
    norm_epsilon = 1e-5


class _Ckpt:
    def __init__(self, mode: str) -> None:
        self.mode = mode
        self.block_interval = 1


def test_checkpointed_model_grads_equal_eager_and_weights_are_tied() -> None:
    """tests/unit/test_gpt_kernels.py:62-78 and test_gpt_model.py:69-88, 278-309 of the reference."""
    torch.manual_seed(0)
    full = R.OracleGPTModel(_Cfg(), activation_checkpoint_config=_Ckpt("full"), dtype=torch.float64)
    torch.manual_seed(0)
    eager = R.OracleGPTModel(_Cfg(), activation_checkpoint_config=_Ckpt("none"), dtype=torch.float64)
    ids = torch.randint(0, 64, (2, 9))
    labels = torch.randint(0, 64, (2, 9))
    lf = full(ids, labels=labels).loss
    le = eager(ids, labels=labels).loss
    lf.backward()
    le.backward()
    torch.testing.assert_close(lf, le)
    assert full.lm_head.weight is full.embedding.weight
    for (n, a), (_, b) in zip(full.named_parameters(), eager.named_parameters()):
        torch.testing.assert_close(a.grad, b.grad, msg=n)
    # full recompute runs each layer forward twice
    assert all(layer.forward_calls == 2 for layer in full.layers)
    assert all(layer.forward_calls == 1 for layer in eager.layers)


# ---------------------------------------------------------------- dropout
def test_splitmix64_known_answers() -> None:
    """Published SplitMix64 outputs (Vigna's splitmix64.c): the first outputs of
    the generator seeded with 0 and with 1234567."""
    import numpy as np

    assert [int(z) for z in R.splitmix64(0, np.arange(4))] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    assert [int(z) for z in R.splitmix64(1234567, np.arange(3))] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423]


def test_dropout_bits_take_the_halves_of_one_draw_per_pair() -> None:
    bits = R.dropout_bits(0, 5)
    assert [int(b) for b in bits[:4]] == [0x7B1DCDAF, 0xE220A839, 0xA1B965F4, 0x6E789E6A]
    assert int(bits[4]) == 0x8009454F


@pytest.mark.parametrize("p", [0.1, 0.5, 0.9])
def test_dropout_keep_rate_and_independence(p) -> None:
    """Keep probability 1 - p within 5 sigma over 2^20 draws; neighbouring
    elements (which share one SplitMix64 output) are uncorrelated; different
    seeds give different masks."""
    n = 1 << 20
    keep = R.dropout_keep(123, (n,), p).float()
    sigma = math.sqrt(p * (1 - p) / n)
    assert abs(float(keep.mean()) - (1 - p)) < 5 * sigma
    a, b = keep[0::2] - keep.mean(), keep[1::2] - keep.mean()
    corr = float((a * b).mean() / (a.square().mean().sqrt() * b.square().mean().sqrt()))
    assert abs(corr) < 5 / math.sqrt(n / 2)
    other = R.dropout_keep(124, (n,), p).float()
    assert float((keep != other).float().mean()) > p * (1 - p)
    assert bool(R.dropout_keep(123, (64,), 0.0).all())


def test_dropout_arithmetic_matches_torch_fp32() -> None:
    """F.dropout's arithmetic: torch's own dropout (native_dropout returns its
    mask) equals dropout_apply with that mask, bit for bit, in fp32."""
    torch.manual_seed(3)
    x = torch.randn(4096)
    for p in (0.1, 0.3, 0.37):
        out, mask = torch.ops.aten.native_dropout(x, p, True)
        assert torch.equal(R.dropout_apply(x, mask, p), out)
    r = torch.randn(4096)
    out, mask = torch.ops.aten.native_dropout(x, 0.2, True)
    assert torch.equal(R.dropout_apply(x, mask, 0.2, residual=r), r + out)


def test_dropout_add_is_unbiased_and_its_own_backward() -> None:
    """E[dropout(x)] = x over seeds (a wrong scale or an inverted mask moves the
    mean by a factor); the backward of residual + dropout(x) through autograd
    of the mask arithmetic is dropout(grad) with the same mask."""
    x = torch.linspace(-2, 2, 64, dtype=torch.float64)
    mean = torch.stack([R.dropout_add(x, 0.25, s) for s in range(4000)]).mean(0)
    torch.testing.assert_close(mean, x, rtol=0.0, atol=0.06)
    xg = x.clone().requires_grad_(True)
    keep = R.dropout_keep(9, x.shape, 0.25)
    (R.dropout_apply(xg, keep, 0.25) * torch.arange(64.0, dtype=torch.float64)).sum().backward()
    expected = R.dropout_apply(torch.arange(64.0, dtype=torch.float64), keep, 0.25)
    torch.testing.assert_close(xg.grad, expected, rtol=1e-12, atol=0.0)


def test_attention_dropout_reduces_to_sdpa_and_is_unbiased() -> None:
    """With a keep-everything mask the dropout path equals the plain SDPA path;
    averaged over seeds it converges to the no-dropout output (unbiased)."""
    torch.manual_seed(4)
    q, k, v = (torch.randn(1, 2, 6, 8, dtype=torch.float64) for _ in range(3))
    plain = R.local_attention(q, k, v, causal=True)
    tiny = R.local_attention(q, k, v, causal=True, dropout_p=1e-12, dropout_seed=5)
    torch.testing.assert_close(tiny, plain, rtol=1e-9, atol=1e-9)
    # a boolean mask (with a fully masked row) and an offset: still the SDPA path's output
    mask = torch.rand(1, 1, 6, 6, generator=torch.Generator().manual_seed(1)) > 0.4
    mask[0, 0, 2] = False
    for causal, offset in ((True, 3), (False, 0)):
        plain_m = R.local_attention(q, k, v, causal=causal, sequence_offset=offset, attention_mask=mask)
        tiny_m = R.local_attention(q, k, v, causal=causal, sequence_offset=offset, attention_mask=mask,
                                   dropout_p=1e-12, dropout_seed=5)
        torch.testing.assert_close(tiny_m, plain_m, rtol=1e-9, atol=1e-9)
        assert torch.count_nonzero(tiny_m[0, :, 2]) == 0
    mean = torch.stack([R.local_attention(q, k, v, causal=True, dropout_p=0.3, dropout_seed=s)
                        for s in range(3000)]).mean(0)
    torch.testing.assert_close(mean, plain, rtol=0.0, atol=0.08)
    # the mask is indexed over [B, Hq, Sq, Sk]: a dropped (b, h, i, j) removes
    # exactly that key's term from that query's output
    keep = R.dropout_keep(11, (1, 2, 6, 6), 0.3)
    probs = torch.softmax((q @ k.transpose(-1, -2)) / math.sqrt(8) + torch.full((6, 6), float("-inf"))
                          .triu(1).to(torch.float64), dim=-1)
    expected = (probs * keep / (1 - float(torch.tensor(0.3, dtype=torch.float32)))) @ v
    got = R.local_attention(q, k, v, causal=True, dropout_p=0.3, dropout_seed=11)
    torch.testing.assert_close(got, expected, rtol=1e-6, atol=1e-6)
