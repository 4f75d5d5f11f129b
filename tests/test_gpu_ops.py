"""Kernel parity on the GPU: each HIP op against the CPU oracle on the same
seeded inputs (fp32: rtol 1e-5; bf16: rtol 2e-2 / atol 1e-2, the atol read
relative to each tensor's largest magnitude and the relative L2 error held to
rtol, tests/parity.py), edge cases (ragged sizes, GQA, offsets, masks, ignored
targets) and determinism."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import nano_megatron_amd as nm
from nano_megatron_amd import functional as Fn
from oracle import reference as R
from parity import assert_close_scaled, assert_loss_close

pytestmark = pytest.mark.gpu


def close(got, exp, dtype, scale_atol=True, msg=""):
    """The dtype's bar with atol scaled to max|exp| (for every tensor, outputs
    and gradients alike; ``scale_atol`` is kept for the call sites)."""
    assert_close_scaled(got, exp, dtype, msg=msg)


def gen(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("rows,cols,dtype", [
    (8192, 1024, torch.bfloat16), (512, 256, torch.float32), (37, 2048, torch.bfloat16),
    (3, 64, torch.float32), (1, 4096, torch.bfloat16),
])
def test_rmsnorm_matches_oracle(device, rows, cols, dtype) -> None:
    g = gen(1)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    w = (1 + 0.02 * torch.randn(cols, generator=g)).to(dtype)
    dy = torch.randn(rows, cols, generator=g).to(dtype)
    xr, wr = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    yr = R.rms_norm(xr, wr, 1e-5)
    yr.backward(dy)
    xd, wd = x.to(device).requires_grad_(True), w.to(device).requires_grad_(True)
    yd = nm.rms_norm(xd, wd, 1e-5)
    yd.backward(dy.to(device))
    close(yd, yr, dtype)
    close(xd.grad, xr.grad, dtype, scale_atol=True)
    close(wd.grad, wr.grad, dtype, scale_atol=True)
    if dtype == torch.bfloat16:
        # forward rounding points replicated: nearly every element bit-equal
        eq = (yd.cpu() == yr).float().mean().item()
        assert eq > 0.99, eq


# ---------------------------------------------------------------- RoPE
@pytest.mark.parametrize("shape,dtype", [
    ((16, 16, 512, 64), torch.bfloat16), ((2, 4, 128, 64), torch.float32),
    ((1, 3, 33, 128), torch.bfloat16),
])
def test_rope_matches_oracle(device, shape, dtype) -> None:
    g = gen(1)
    b, h, s, d = shape
    q = torch.randn(b, s, h, d, generator=g).to(dtype).transpose(1, 2)
    k = torch.randn(b, s, max(1, h // 2), d, generator=g).to(dtype).transpose(1, 2)
    cos, sin = R.rope_cos_sin(torch.arange(s), d, 1e4, dtype)
    qr, kr = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    oq, ok = R.apply_rotary_pos_emb(qr, kr, cos, sin)
    gq, gk = torch.randn_like(oq), torch.randn_like(ok)
    (oq * gq).sum().backward(retain_graph=True)
    (ok * gk).sum().backward()
    rope = nm.RotaryEmbedding(d)
    dcos, dsin = rope(torch.arange(s, device=device), dtype=dtype)
    close(dcos, cos, dtype)
    qd, kd = q.to(device).requires_grad_(True), k.to(device).requires_grad_(True)
    pq, pk = nm.apply_rotary_pos_emb(qd, kd, dcos, dsin)
    (pq * gq.to(device)).sum().backward(retain_graph=True)
    (pk * gk.to(device)).sum().backward()
    close(pq, oq, dtype)
    close(pk, ok, dtype)
    close(qd.grad, qr.grad, dtype)
    close(kd.grad, kr.grad, dtype)


@pytest.mark.parametrize("d", [64, 128])
def test_rope_bf16_forward_is_bit_exact(device, d) -> None:
    """Given the same bf16 cos/sin tables, the kernel rounds where the reference's
    three bf16 tensor ops round (q*cos, rotate_half(q)*sin, their sum), so the
    rotated q and k are bit-equal to the oracle's (nn/rotary.py:27-38)."""
    g = gen(5)
    b, h, s = 2, 4, 96
    q = torch.randn(b, s, h, d, generator=g).to(torch.bfloat16).transpose(1, 2)
    k = torch.randn(b, s, h // 2, d, generator=g).to(torch.bfloat16).transpose(1, 2)
    # positions far from 0, so cos/sin take many distinct values
    cos, sin = R.rope_cos_sin(torch.arange(s) + 3000, d, 1e4, torch.bfloat16)
    oq, ok = R.apply_rotary_pos_emb(q, k, cos, sin)
    pq, pk = nm.apply_rotary_pos_emb(q.to(device), k.to(device), cos.to(device), sin.to(device))
    assert torch.equal(pq.cpu(), oq)
    assert torch.equal(pk.cpu(), ok)


def test_rope_offset_positions_and_inverse(device) -> None:
    """Offset form (positions offset + s) equals explicit ids; inverse undoes forward."""
    g = gen(2)
    x = torch.randn(2, 40, 3, 64, generator=g).to(device)
    tab = Fn.RopeTables.get(device, 64, 1e4, 200)
    a = torch.empty_like(x)
    Fn.rope_apply(x, a, tab.cos, tab.sin, pos_offset=100)
    pos = torch.arange(100, 140, dtype=torch.int32, device=device)
    b = torch.empty_like(x)
    Fn.rope_apply(x, b, tab.cos, tab.sin, positions=pos)
    assert torch.equal(a, b)
    back = torch.empty_like(x)
    Fn.rope_apply(a, back, tab.cos, tab.sin, pos_offset=100, inverse=True)
    torch.testing.assert_close(back, x, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- SwiGLU
@pytest.mark.parametrize("rows,cols,dtype", [
    (8192, 2736, torch.bfloat16), (512, 688, torch.float32), (13, 5632, torch.bfloat16),
])
def test_swiglu_matches_oracle(device, rows, cols, dtype) -> None:
    g0 = gen(1)
    gate = torch.randn(rows, cols, generator=g0).to(dtype)
    up = torch.randn(rows, cols, generator=g0).to(dtype)
    dh = torch.randn(rows, cols, generator=g0).to(dtype)
    gr, ur = gate.clone().requires_grad_(True), up.clone().requires_grad_(True)
    hr = R.swiglu(gr, ur)
    hr.backward(dh)
    gd, ud = gate.to(device).requires_grad_(True), up.to(device).requires_grad_(True)
    hd = nm.swiglu(gd, ud)
    hd.backward(dh.to(device))
    close(hd, hr, dtype)
    close(gd.grad, gr.grad, dtype, scale_atol=True)
    close(ud.grad, ur.grad, dtype, scale_atol=True)
    # fused recompute-backward re-emits h bit-identically to the forward
    dg, du, h2 = (torch.empty_like(gd) for _ in range(3))
    Fn.swiglu_bwd(gd.detach(), ud.detach(), dh.to(device), dg, du, h2)
    assert torch.equal(h2, hd.detach())


@pytest.mark.gpu
def test_swiglu_activation_exact_for_every_bf16_gate(device) -> None:
    """silu(g) rounded to bf16 equals the exact formula g / (1 + exp(-g)) (fp32,
    IEEE division, evaluated by torch on the same GPU) for every finite bf16
    gate value, in the forward kernel and as re-emitted by the backward: the
    kernels' fast sigmoid is used only where it rounds the same way, and the
    gate is a bf16 value wherever that function runs, so this covers every
    input it can see."""
    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    g = bits.view(torch.bfloat16)
    g = g[torch.isfinite(g.float())].reshape(255, 256).to(device)
    up = torch.ones_like(g)
    h = Fn.swiglu_fwd(g, up)
    gf = g.float()
    exact = (gf / (1.0 + torch.exp(-gf))).to(torch.bfloat16)
    mismatch = (h != exact).sum().item()
    assert mismatch == 0, f"{mismatch} gate values round differently from the exact formula"
    dg, du, h2 = (torch.empty_like(g) for _ in range(3))
    Fn.swiglu_bwd(g, up, torch.ones_like(g), dg, du, h2)
    assert torch.equal(h2, exact)


# ---------------------------------------------------------------- attention
ATTN_CASES = [
    # b, hq, hkv, sq, sk, d, dtype, offset, causal
    (2, 4, 4, 128, 128, 64, torch.bfloat16, 0, True),
    (1, 4, 2, 200, 200, 64, torch.bfloat16, 0, True),
    (1, 2, 2, 96, 96, 128, torch.bfloat16, 0, True),
    (1, 4, 4, 64, 80, 64, torch.bfloat16, 0, False),
    (1, 2, 1, 64, 128, 64, torch.bfloat16, 64, True),
    (2, 4, 2, 100, 100, 64, torch.float32, 0, True),
    (1, 2, 2, 48, 112, 64, torch.float32, 64, True),
    (1, 8, 2, 256, 256, 128, torch.bfloat16, 0, True),
    # head dim 128: two 256-query workgroups with a ragged tail, GQA; and an offset
    # query block over a longer key range (ring share shape)
    (1, 4, 2, 300, 300, 128, torch.bfloat16, 0, True),
    (2, 2, 2, 130, 260, 128, torch.bfloat16, 130, True),
    # head dim 64 from 1024 queries (two column tiles per wave, three workgroups per CU),
    # ragged last tile
    (1, 2, 2, 1100, 1100, 64, torch.bfloat16, 0, True),
    # config-4 attention: GQA 4:1 at head dim 64 over 2048 queries (the C4 heads,
    # 32 query / 8 KV, at batch 1), and the same ratio with a ragged tail
    (1, 8, 2, 2048, 2048, 64, torch.bfloat16, 0, True),
    (1, 32, 8, 2048, 2048, 64, torch.bfloat16, 0, True),
    (1, 8, 2, 1100, 1100, 64, torch.bfloat16, 0, True),
    # tiles mostly padding: one query and one key, a 17-token sequence; GQA 8:1;
    # more queries than keys without the causal mask at head dim 128
    (1, 2, 2, 1, 1, 64, torch.bfloat16, 0, True),
    (2, 4, 4, 17, 17, 64, torch.bfloat16, 0, True),
    (3, 2, 2, 33, 33, 128, torch.bfloat16, 0, True),
    (1, 16, 2, 96, 96, 64, torch.bfloat16, 0, True),
    (1, 2, 1, 200, 64, 128, torch.bfloat16, 0, False),
    # 512-1023 queries at head dim 64 (eight waves of four column tiles, each
    # column tile storing its output at its last key tile): an offset query
    # block over a ragged key range, and the non-causal case (every tile stores
    # at the last key tile)
    (1, 4, 2, 700, 764, 64, torch.bfloat16, 64, True),
    (1, 2, 2, 600, 600, 64, torch.bfloat16, 0, False),
]


@pytest.mark.parametrize("b,hq,hkv,sq,sk,d,dtype,offset,causal", ATTN_CASES)
def test_attention_matches_oracle(device, b, hq, hkv, sq, sk, d, dtype, offset, causal) -> None:
    g = gen(1)
    q = torch.randn(b, hq, sq, d, generator=g).to(dtype)
    k = torch.randn(b, hkv, sk, d, generator=g).to(dtype)
    v = torch.randn(b, hkv, sk, d, generator=g).to(dtype)
    do = torch.randn(b, hq, sq, d, generator=g).to(dtype)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    if causal:
        # SDPA's offset mask uses key positions 0..Sk-1 and query positions offset + i
        o_ref = R.local_attention(qr, kr, vr, causal=True, sequence_offset=offset)
    else:
        o_ref = R.local_attention(qr, kr, vr, causal=False)
    o_ref.backward(do)
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    o = nm.attention(qd, kd, vd, causal=causal, sequence_offset=offset)
    o.backward(do.to(device))
    close(o, o_ref, dtype)
    close(qd.grad, qr.grad, dtype, scale_atol=True, msg="dq")
    close(kd.grad, kr.grad, dtype, scale_atol=True, msg="dk")
    close(vd.grad, vr.grad, dtype, scale_atol=True, msg="dv")


@pytest.mark.parametrize("hq,hkv,sq,sk,d", [(4, 2, 64, 320, 64), (4, 1, 100, 400, 128)])
def test_attention_keys_past_every_query(device, hq, hkv, sq, sk, d) -> None:
    """Causal attention at offset 0 with more keys than queries: keys past the
    last query position are seen by no query, so whole 128-key tiles have an
    empty query-tile stream in the dK/dV kernel (alone or as the second key
    tile of a work item).  Their dK and dV are exactly zero, and everything
    matches the oracle within the bf16 bars."""
    g = gen(3)
    q = torch.randn(1, hq, sq, d, generator=g).bfloat16()
    k = torch.randn(1, hkv, sk, d, generator=g).bfloat16()
    v = torch.randn(1, hkv, sk, d, generator=g).bfloat16()
    do = torch.randn(1, hq, sq, d, generator=g).bfloat16()
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    o_ref = R.local_attention(qr, kr, vr, causal=True, sequence_offset=0)
    o_ref.backward(do)
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    o = nm.attention(qd, kd, vd, causal=True, sequence_offset=0)
    o.backward(do.to(device))
    close(o, o_ref, torch.bfloat16)
    close(qd.grad, qr.grad, torch.bfloat16, scale_atol=True, msg="dq")
    close(kd.grad, kr.grad, torch.bfloat16, scale_atol=True, msg="dk")
    close(vd.grad, vr.grad, torch.bfloat16, scale_atol=True, msg="dv")
    assert torch.count_nonzero(kd.grad[:, :, sq:].cpu()) == 0
    assert torch.count_nonzero(vd.grad[:, :, sq:].cpu()) == 0
    assert torch.count_nonzero(kd.grad[:, :, :sq].cpu()) > 0


MASK_CASES = [
    # (dtype, causal, offset, kind, hq, hkv, sq, sk, d)
    (torch.bfloat16, True, 0, "bool", 4, 2, 64, 64, 64),
    (torch.bfloat16, True, 7, "bool", 4, 4, 37, 45, 128),
    (torch.bfloat16, False, 0, "add", 4, 1, 33, 50, 64),
    (torch.float32, True, 0, "bool", 2, 2, 40, 40, 32),
    (torch.float32, False, 0, "add", 4, 2, 29, 31, 80),
]


@pytest.mark.parametrize("dtype,causal,offset,kind,hq,hkv,sq,sk,d", MASK_CASES)
def test_masked_attention_matches_oracle(device, dtype, causal, offset, kind, hq, hkv, sq, sk, d) -> None:
    """local_attention with attention_mask through the HIP backend (nmb_attn_masked_*)
    against the oracle (torch_backend.py:60-76): a boolean mask [B, 1, Sq, Sk]
    ANDed with the causal mask, with one query row fully masked (zero output and
    gradients), or an additive mask [Sq, Sk] of the query dtype with -inf
    entries; GQA, head dims 32-128, ragged lengths; forward and q/k/v gradients."""
    g = gen(7)
    b = 2
    q = torch.randn(b, hq, sq, d, generator=g).to(dtype)
    k = torch.randn(b, hkv, sk, d, generator=g).to(dtype)
    v = torch.randn(b, hkv, sk, d, generator=g).to(dtype)
    do = torch.randn(b, hq, sq, d, generator=g).to(dtype)
    if kind == "bool":
        mask = torch.rand(b, 1, sq, sk, generator=g) > 0.3
        mask[1, 0, 3] = False
    else:
        mask = torch.randn(sq, sk, generator=g).to(dtype)
        mask[2, 1:9] = float("-inf")
    qr, kr, vr = (t.float().clone().requires_grad_(True) for t in (q, k, v))
    mr = mask if kind == "bool" else mask.float()
    o_ref = R.local_attention(qr, kr, vr, causal=causal, sequence_offset=offset, attention_mask=mr)
    o_ref.backward(do.float())
    backend = nm.HipKernelBackend()
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    o = backend.local_attention(qd, kd, vd, causal=causal, sequence_offset=offset, attention_mask=mask.to(device))
    o.backward(do.to(device))
    close(o, o_ref, dtype)
    close(qd.grad, qr.grad, dtype, scale_atol=True, msg="dq")
    close(kd.grad, kr.grad, dtype, scale_atol=True, msg="dk")
    close(vd.grad, vr.grad, dtype, scale_atol=True, msg="dv")
    if kind == "bool":
        assert torch.count_nonzero(o[1, :, 3]) == 0 and torch.count_nonzero(qd.grad[1, :, 3]) == 0


def test_masked_attention_rejects_what_the_reference_rejects(device) -> None:
    q = torch.randn(1, 2, 8, 64, device=device, dtype=torch.bfloat16)
    backend = nm.HipKernelBackend()
    with pytest.raises(ValueError, match="boolean"):  # `mask & causal_mask` needs a boolean mask
        backend.local_attention(q, q, q, causal=True, attention_mask=torch.zeros(8, 8, device=device,
                                                                                  dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="broadcast"):
        backend.local_attention(q, q, q, causal=False, attention_mask=torch.ones(3, 8, 8, device=device,
                                                                                  dtype=torch.bool))
    with pytest.raises(ValueError, match="dtype"):
        backend.local_attention(q, q, q, causal=False, attention_mask=torch.zeros(8, 8, device=device))


def test_attention_c3_shape_and_lse(device) -> None:
    """Config 3 attention shape [16,16,512,64] bf16, forward and backward against
    the oracle; lse == logsumexp of masked scores."""
    g = gen(1)
    b, h, s, d = 16, 16, 512, 64
    q = torch.randn(b, s, h, d, generator=g).bfloat16()
    k = torch.randn(b, s, h, d, generator=g).bfloat16()
    v = torch.randn(b, s, h, d, generator=g).bfloat16()
    do = torch.randn(b, s, h, d, generator=g).bfloat16()
    o, lse = Fn.attn_fwd_bshd(q.to(device), [k.to(device)], [v.to(device)], (0,), causal=True,
                              q_offset=0, scale=None)
    qr, kr, vr = (t.transpose(1, 2).clone().requires_grad_(True) for t in (q, k, v))
    ref = R.local_attention(qr, kr, vr)
    ref.backward(do.transpose(1, 2))
    close(o.transpose(1, 2), ref, torch.bfloat16)
    # the backward as the model runs it (delta fused in the dQ kernel, then dK/dV)
    qd, kd, vd = (t.to(device).transpose(1, 2).requires_grad_(True) for t in (q, k, v))
    od = nm.attention(qd, kd, vd)
    od.backward(do.to(device).transpose(1, 2))
    assert torch.equal(od.detach().transpose(1, 2), o)
    close(qd.grad, qr.grad, torch.bfloat16, scale_atol=True, msg="dq")
    close(kd.grad, kr.grad, torch.bfloat16, scale_atol=True, msg="dk")
    close(vd.grad, vr.grad, torch.bfloat16, scale_atol=True, msg="dv")
    qf, kf = q[:2].float().transpose(1, 2), k[:2].float().transpose(1, 2)
    scores = qf @ kf.transpose(-1, -2) / math.sqrt(d)
    mask = torch.ones(s, s, dtype=torch.bool).tril()
    ref_lse = scores.masked_fill(~mask, -math.inf).logsumexp(-1)
    torch.testing.assert_close(lse[:2].cpu(), ref_lse, rtol=1e-3, atol=2e-3)


def test_attention_is_deterministic(device) -> None:
    g = gen(3)
    q, k, v, do = (torch.randn(2, 8, 256, 64, generator=g).bfloat16().to(device) for _ in range(4))
    outs = []
    for _ in range(2):
        qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
        o = nm.attention(qd, kd, vd)
        o.backward(do)
        outs.append((o.detach(), qd.grad, kd.grad, vd.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("d,dtype", [(128, torch.bfloat16), (64, torch.float32)])
def test_ring_share_matches_oracle(device, d, dtype) -> None:
    """One rank (r=3 of 4) of the ring: blocks visited (3 - s) % 4, block-causal."""
    g = gen(1)
    s, h, hkv, rank = 192, 4, 2, 3
    q = torch.randn(1, h, s, d, generator=g).to(dtype)
    blocks = [(torch.randn(1, hkv, s, d, generator=g).to(dtype), torch.randn(1, hkv, s, d, generator=g).to(dtype))
              for _ in range(4)]
    order = [(rank - step) % 4 for step in range(4)]
    offsets = [r * s for r in order]
    kvs = [blocks[r] for r in order]
    out_ref, lse_ref = R.ring_attention_forward(q, kvs, offsets, causal=True, query_offset=rank * s)
    do = torch.randn(1, h, s, d, generator=g).to(dtype)
    dq_ref, dk_ref, dv_ref = R.ring_attention_backward(do, q, kvs, offsets, out_ref, lse_ref,
                                                       causal=True, query_offset=rank * s)
    qd = q.to(device).requires_grad_(True)
    kd = [(k.to(device).requires_grad_(True), v.to(device).requires_grad_(True)) for k, v in kvs]
    o = nm.ring_attention(qd, kd, offsets, causal=True, query_offset=rank * s)
    o.backward(do.to(device))
    close(o, out_ref, dtype)
    close(qd.grad, dq_ref, dtype, scale_atol=True)
    for (k, v), dk, dv in zip(kd, dk_ref, dv_ref):
        close(k.grad, dk, dtype, scale_atol=True)
        close(v.grad, dv, dtype, scale_atol=True)


# ---------------------------------------------------------------- LM head + CE
@pytest.mark.parametrize("rows,hidden,vocab,dtype,chunk", [
    (512, 256, 8192, torch.float32, 200), (1024, 1024, 8192, torch.bfloat16, 384),
    (64, 128, 1000, torch.float32, 64),
])
def test_lm_head_cross_entropy_matches_oracle(device, rows, hidden, vocab, dtype, chunk) -> None:
    g = gen(1)
    x = torch.randn(rows, hidden, generator=g).to(dtype)
    e = (0.02 * torch.randn(vocab, hidden, generator=g)).to(dtype)
    t = torch.randint(0, vocab, (rows,), generator=g)
    t[::7] = -100
    xr, er = x.clone().requires_grad_(True), e.clone().requires_grad_(True)
    lr = R.cross_entropy_tokens(torch.nn.functional.linear(xr, er), t, reduction="mean")
    lr.backward()
    xd, ed = x.to(device).requires_grad_(True), e.to(device).requires_grad_(True)
    ld = nm.lm_head_cross_entropy(xd, ed, t.to(device), chunk=chunk)
    ld.backward()
    assert_loss_close(ld, lr, dtype)
    close(xd.grad, xr.grad, dtype, msg="dx")
    close(ed.grad, er.grad, dtype, msg="dE")
    per_tok = nm.lm_head_cross_entropy(xd.detach(), ed.detach(), t.to(device), reduction="none", chunk=chunk)
    assert torch.all(per_tok.cpu()[t == -100] == 0)
    with pytest.raises(ValueError, match="outside"):
        nm.lm_head_cross_entropy(xd.detach(), ed.detach(), torch.full_like(t, vocab).to(device))


@pytest.mark.parametrize("reduction", ["sum", "mean"])
def test_lm_head_cross_entropy_c2_bf16(device, reduction) -> None:
    """Config 2's chunked cross entropy, [8192, 1024] x [1024, 8192] in bf16
    (x ~ N(0, 1), E ~ N(0, 0.02), seed 1, uniform labels): with reduction
    "sum" the logits' gradient is softmax - onehot per token, so dE is O(1)
    and dX ~ 2e-2; the loss within rtol 1e-3 and dX, dE within the bf16 bar
    scaled to each tensor, against the oracle's bf16 path (bf16 logits, fp32
    softmax, the gradient cast to bf16: tensor_parallel/cross_entropy.py:
    30-86, tests/unit/test_tensor_parallel_layers.py:139-166)."""
    g = gen(1)
    x = torch.randn(8192, 1024, generator=g).bfloat16()
    e = (0.02 * torch.randn(8192, 1024, generator=g)).bfloat16()
    t = torch.randint(0, 8192, (8192,), generator=g)
    xr, er = x.clone().requires_grad_(True), e.clone().requires_grad_(True)
    lr = R.cross_entropy_tokens(torch.nn.functional.linear(xr, er), t, reduction=reduction)
    lr.backward()
    xd, ed = x.to(device).requires_grad_(True), e.to(device).requires_grad_(True)
    ld = nm.lm_head_cross_entropy(xd, ed, t.to(device), reduction=reduction)
    ld.backward()
    assert_loss_close(ld, lr, torch.bfloat16)
    close(xd.grad, xr.grad, torch.bfloat16, msg="dx")
    close(ed.grad, er.grad, torch.bfloat16, msg="dE")
    if reduction == "sum":
        assert float(er.grad.float().abs().max()) > 0.5  # O(1): a bar that a zeroed dE cannot pass


# ---------------------------------------------------------------- GEMM
@pytest.mark.parametrize("m,n,k,layout", [
    (512, 384, 256, "NT"), (1000, 264, 200, "NT"), (333, 520, 136, "NN"),
    (520, 88, 72, "TN"), (256, 1024, 4096, "TN"), (300, 256, 64, "NN"),
    # one row, one 8-column group, the smallest K; 7 rows; a long K over a
    # narrow product (K split into fp32 partials)
    (1, 8, 8, "NT"), (7, 16, 24, "NT"), (64, 8, 4104, "TN"), (8, 40, 8200, "NN"),
])
def test_gemm_bf16_matches_fp32_product(device, m, n, k, layout) -> None:
    """nmb_gemm_bf16 for row/column-major operand mixes, ragged tiles, alpha/beta."""
    g = torch.Generator(device=device).manual_seed(m + n + k)
    bf = torch.bfloat16
    if layout == "NT":
        a, b = torch.randn(m, k, device=device, generator=g).to(bf), torch.randn(n, k, device=device, generator=g).to(bf).t()
    elif layout == "NN":
        a, b = torch.randn(m, k, device=device, generator=g).to(bf), torch.randn(k, n, device=device, generator=g).to(bf)
    else:
        a, b = torch.randn(k, m, device=device, generator=g).to(bf).t(), torch.randn(k, n, device=device, generator=g).to(bf)
    c = torch.randn(m, n, device=device, generator=g).to(bf)
    ref = 0.5 * (a.float() @ b.float()) + 2.0 * c.float()
    out = Fn.mm(a, b, c=c, alpha=0.5, beta=2.0)
    torch.testing.assert_close(out.float(), ref, rtol=2e-2, atol=2e-2 * float(ref.abs().max()))
    out2 = Fn.mm(a, b)
    torch.testing.assert_close(out2.float(), a.float() @ b.float(), rtol=2e-2,
                               atol=2e-2 * float((a.float() @ b.float()).abs().max()))


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k,layout", [
    (4100, 2056, 512, "NT"), (8192, 1032, 1024, "NN"), (2056, 4104, 264, "NN"), (3000, 5472, 1024, "NT"),
])
def test_gemm_bf16_many_tiles_per_workgroup(device, m, n, k, layout) -> None:
    """Products with more output tiles than resident workgroups (each workgroup
    then computes several tiles back to back), ragged edges and a K tail."""
    g = torch.Generator(device=device).manual_seed(m * 7 + n + k)
    bf = torch.bfloat16
    a = torch.randn(m, k, device=device, generator=g).to(bf)
    b = (torch.randn(n, k, device=device, generator=g).to(bf).t() if layout == "NT"
         else torch.randn(k, n, device=device, generator=g).to(bf))
    ref = a.float() @ b.float()
    out = Fn.mm(a, b)
    torch.testing.assert_close(out.float(), ref, rtol=2e-2, atol=2e-2 * float(ref.abs().max()))
    # the same product twice gives the same bits
    assert torch.equal(Fn.mm(a, b), out)


@pytest.mark.gpu
@pytest.mark.parametrize("m,f,h", [(8192, 2736, 1024), (4096, 5632, 2048), (300, 200, 136)])
def test_gemm_swiglu_bwd_equals_gemm_then_swiglu_bwd(device, m, f, h) -> None:
    """nmb_gemm_bf16_swiglu_bwd (ds = dY Wd with the SwiGLU backward as the
    epilogue) against the product then nmb_swiglu_bwd: bit for bit where both
    use unsplit plans (M >= 4096), and against the fp32 expression."""
    g = torch.Generator(device=device).manual_seed(m + f + h)
    bf = torch.bfloat16
    dy = torch.randn(m, h, device=device, generator=g).to(bf)
    wd = (0.05 * torch.randn(h, f, device=device, generator=g)).to(bf)
    gu = torch.randn(m, 2 * f, device=device, generator=g).to(bf)
    dgu, act = Fn.mm_swiglu_bwd(dy, wd, gu)
    dgu2, none = Fn.mm_swiglu_bwd(dy, wd, gu, act=False)
    assert none is None and torch.equal(dgu, dgu2)
    ds = Fn.mm(dy, wd)
    rdgu = torch.empty_like(gu)
    ract = torch.empty(m, f, dtype=bf, device=device)
    Fn.swiglu_bwd(gu[:, :f], gu[:, f:], ds, rdgu[:, :f], rdgu[:, f:], ract)
    assert torch.equal(act, ract)
    if m >= 4096:
        assert torch.equal(dgu, rdgu)
    gf, uf = gu[:, :f].float(), gu[:, f:].float()
    dsf = dy.float() @ wd.float()
    sig = torch.sigmoid(gf)
    torch.testing.assert_close(dgu[:, f:].float(), dsf * gf * sig, rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(dgu[:, :f].float(), dsf * uf * sig * (1 + gf * (1 - sig)), rtol=2e-2, atol=2e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("batch,seq,hq,hkv,d,offset,explicit", [
    (4, 128, 4, 2, 64, 0, False),
    (2, 256, 2, 1, 128, 0, True),
    (3, 64, 4, 4, 64, 37, False),
])
def test_gemm_rope_equals_gemm_then_rope(device, batch, seq, hq, hkv, d, offset, explicit) -> None:
    """nmb_gemm_bf16_rope == nmb_gemm_bf16 followed by the rotary kernel on q and k, bit for bit."""
    import nano_megatron_amd as nm

    g = torch.Generator(device=device).manual_seed(seq + d + offset)
    bf = torch.bfloat16
    hidden = 256
    n = (hq + 2 * hkv) * d
    x = torch.randn(batch * seq, hidden, device=device, generator=g).to(bf)
    w = (0.05 * torch.randn(n, hidden, device=device, generator=g)).to(bf)
    tab = nm.RotaryEmbedding(d).tables(device, 1024)
    positions = None
    if explicit:
        positions = torch.stack([torch.randperm(1024, device=device, generator=g)[:seq] for _ in range(batch)])
        positions = positions.to(torch.int32)
    rope_cols = (hq + hkv) * d
    fused = Fn.mm_rope(x, w.t(), seq=seq, head_dim=d, rope_cols=rope_cols, cos=tab.cos, sin=tab.sin,
                       pos_offset=offset, positions=positions)
    ref = Fn.mm(x, w.t())
    qk = ref.view(batch, seq, n)[:, :, :rope_cols].unflatten(2, (hq + hkv, d))
    Fn.rope_apply(qk, qk, tab.cos, tab.sin, pos_offset=offset, positions=positions)
    assert torch.equal(fused, ref)
    # and against the fp32 product, rotated in fp32 (tolerance of the bf16 roundings)
    ref32 = (x.float() @ w.float().t()).view(batch, seq, n)
    pos = positions.long() if positions is not None else (offset + torch.arange(seq, device=device)).expand(batch, seq)
    inv = 1.0 / (1e4 ** (torch.arange(0, d, 2, device=device).float() / d))
    f = pos[..., None].float() * inv
    cos, sin = torch.cat([f, f], -1).cos()[:, :, None], torch.cat([f, f], -1).sin()[:, :, None]
    q = ref32[:, :, :rope_cols].unflatten(2, (hq + hkv, d))
    rot = torch.cat([-q[..., d // 2:], q[..., : d // 2]], -1)
    exp = ref32.clone()
    exp[:, :, :rope_cols] = (q * cos + rot * sin).flatten(2)
    torch.testing.assert_close(fused.view(batch, seq, n).float(), exp, rtol=2e-2, atol=2e-2)


@pytest.mark.gpu
# config-3 rows: neither the fused entry nor the reference GEMM splits K there
@pytest.mark.parametrize("batch,seq,heads,hidden,explicit,b_rowmajor", [(16, 512, 16, 1024, False, False),
                                                                        (4, 2048, 16, 1024, True, False),
                                                                        (16, 512, 16, 1024, False, True)])
def test_gemm_rope_split_launch_equals_gemm_then_rope(device, batch, seq, heads, hidden, explicit,
                                                      b_rowmajor) -> None:
    """At the config-3 Q/K/V shape the entry point runs the q/k columns (RoPE, 256 x
    256 tiles) and the v columns (plain product, 256 x 128 tiles) in one launch
    (gemm_pair_kernel); the result still equals one GEMM followed by the rotary
    kernel, bit for bit, with offset or explicit per-token positions."""
    import nano_megatron_amd as nm

    g = torch.Generator(device=device).manual_seed(11)
    bf = torch.bfloat16
    d = hidden // heads
    n = 3 * hidden
    x = torch.randn(batch * seq, hidden, device=device, generator=g).to(bf)
    w = (0.05 * torch.randn(n, hidden, device=device, generator=g)).to(bf)
    tab = nm.RotaryEmbedding(d).tables(device, 2 * seq)
    pos = (torch.randint(0, 2 * seq, (batch, seq), device=device, generator=g).to(torch.int32)
           if explicit else None)
    wt = w.t().contiguous() if b_rowmajor else w.t()  # B as [K, N] row-major or the weight's W^T view
    fused = Fn.mm_rope(x, wt, seq=seq, head_dim=d, rope_cols=2 * hidden, cos=tab.cos, sin=tab.sin,
                       positions=pos)
    ref = Fn.mm(x, wt)
    qk = ref.view(batch, seq, n)[:, :, :2 * hidden].unflatten(2, (2 * heads, d))
    Fn.rope_apply(qk, qk, tab.cos, tab.sin, positions=pos)
    assert torch.equal(fused, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("m,f,k,scale", [
    (8192, 2736, 1024, 1.0),  # the config-3 gate/up shape (F not a multiple of 128)
    (512, 2736, 1024, 1.0),
    (300, 200, 256, 1.0),     # ragged rows and columns, small-tile configuration
    (1000, 1032, 520, 8.0),   # ragged K; large gates reach silu's exact-formula branches
])
def test_gemm_swiglu_equals_gemm_then_swiglu(device, m, f, k, scale) -> None:
    """nmb_gemm_bf16_swiglu: the activation equals nmb_swiglu_fwd of the product it
    writes, bit for bit; the product is the same bits with or without the
    activation; both match the fp32 expression."""
    g = torch.Generator(device=device).manual_seed(m + f + k)
    bf = torch.bfloat16
    x = (scale * torch.randn(m, k, device=device, generator=g)).to(bf)
    w = (0.05 * torch.randn(2 * f, k, device=device, generator=g)).to(bf)
    act, _ = Fn.mm_gate_up(x, w, act=True, gu=False)
    _, gu = Fn.mm_gate_up(x, w, act=False, gu=True)
    act2, gu2 = Fn.mm_gate_up(x, w, act=True, gu=True)
    ref = Fn.swiglu_fwd(gu[:, :f], gu[:, f:])
    assert torch.equal(act, ref) and torch.equal(act2, ref) and torch.equal(gu2, gu)
    if m >= 4096:  # unsplit plans on both sides: the plain GEMM gives the same product
        assert torch.equal(gu, Fn.mm(x, w.t()))
    p = x.float() @ w.float().t()
    torch.testing.assert_close(gu.float(), p, rtol=1e-2, atol=1e-2 * scale)
    exp = torch.nn.functional.silu(p[:, :f]) * p[:, f:]
    torch.testing.assert_close(act.float(), exp, rtol=2e-2, atol=2e-2 * scale * scale)
    # outputs with row strides wider than F and 2F
    wide = torch.full((m, f + 24), 7.0, dtype=bf, device=device)
    wide_gu = torch.full((m, 2 * f + 8), 7.0, dtype=bf, device=device)
    Fn.mm_gate_up(x, w, act=True, gu=True, act_out=wide[:, :f], gu_out=wide_gu[:, :2 * f])
    assert torch.equal(wide[:, :f], ref) and bool((wide[:, f:] == 7.0).all())
    assert torch.equal(wide_gu[:, :2 * f], gu) and bool((wide_gu[:, 2 * f:] == 7.0).all())


@pytest.mark.gpu
@pytest.mark.parametrize("batch,seq,hq,hkv,d,offset,explicit", [
    (2, 256, 4, 4, 64, 0, False),
    (2, 192, 4, 2, 64, 5, False),
    (1, 128, 2, 1, 128, 0, True),
])
def test_attn_bwd_rope_equals_bwd_then_rope(device, batch, seq, hq, hkv, d, offset, explicit) -> None:
    """nmb_attn_bwd_rope == nmb_attn_bwd followed by the inverse rotary kernel on dq and dk, bit for bit."""
    import nano_megatron_amd as nm

    g = torch.Generator(device=device).manual_seed(seq * d + offset)
    bf = torch.bfloat16
    qkv = torch.randn(batch, seq, (hq + 2 * hkv) * d, device=device, generator=g).to(bf)
    q = qkv[:, :, : hq * d].unflatten(2, (hq, d))
    k = qkv[:, :, hq * d : (hq + hkv) * d].unflatten(2, (hkv, d))
    v = qkv[:, :, (hq + hkv) * d :].unflatten(2, (hkv, d))
    o, lse = Fn.attn_fwd_bshd(q, [k], [v], (0,), causal=True, q_offset=offset, scale=None)
    do = torch.randn(batch, seq, hq, d, device=device, generator=g).to(bf)
    tab = nm.RotaryEmbedding(d).tables(device, 1024)
    positions = None
    if explicit:
        positions = torch.stack([torch.randperm(1024, device=device, generator=g)[:seq] for _ in range(batch)])
        positions = positions.to(torch.int32)
    grads = []
    for fused in (True, False):
        dqkv = torch.empty_like(qkv)
        dq = dqkv[:, :, : hq * d].unflatten(2, (hq, d))
        dk = dqkv[:, :, hq * d : (hq + hkv) * d].unflatten(2, (hkv, d))
        dv = dqkv[:, :, (hq + hkv) * d :].unflatten(2, (hkv, d))
        if fused:
            Fn.attn_bwd_rope_bshd(q, k, v, o, do, lse, dq, dk, dv, causal=True, q_offset=offset, scale=None,
                                  cos=tab.cos, sin=tab.sin, pos_offset=offset, positions=positions)
        else:
            Fn.attn_bwd_bshd(q, [k], [v], (0,), o, do, lse, dq, [dk], [dv], causal=True, q_offset=offset,
                             scale=None)
            Fn.rope_apply(dq, dq, tab.cos, tab.sin, pos_offset=offset, positions=positions, inverse=True)
            Fn.rope_apply(dk, dk, tab.cos, tab.sin, pos_offset=offset, positions=positions, inverse=True)
        grads.append(dqkv)
    assert torch.equal(grads[0], grads[1])


@pytest.mark.gpu
@pytest.mark.parametrize("b,s,hq,hkv,d,causal,blocks", [
    (2, 512, 4, 4, 64, True, 1),
    (1, 300, 8, 2, 64, True, 1),
    (2, 256, 4, 4, 64, False, 1),
    (1, 256, 2, 2, 128, True, 1),
    (1, 128, 2, 1, 128, True, 3),
])
def test_attn_fwd_from_lse_matches_forward(device, b, s, hq, hkv, d, causal, blocks) -> None:
    """O recomputed from the saved LSE equals the forward's O (bf16 tolerance)."""
    g = torch.Generator(device=device).manual_seed(s + d + blocks)
    bf = torch.bfloat16
    q = torch.randn(b, s, hq, d, device=device, generator=g).to(bf)
    ks = [torch.randn(b, s, hkv, d, device=device, generator=g).to(bf) for _ in range(blocks)]
    vs = [torch.randn(b, s, hkv, d, device=device, generator=g).to(bf) for _ in range(blocks)]
    offs = tuple(i * s for i in range(blocks))
    q_offset = (blocks - 1) * s
    o, lse = Fn.attn_fwd_bshd(q, ks, vs, offs, causal=causal, q_offset=q_offset, scale=None)
    o2 = Fn.attn_fwd_from_lse_bshd(q, ks, vs, offs, lse, causal=causal, q_offset=q_offset, scale=None)
    torch.testing.assert_close(o2.float(), o.float(), rtol=2e-2, atol=1e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("vocab,hidden,tokens", [(1000, 256, 4096), (8192, 1024, 8192), (37, 1088, 300)])
def test_embedding_matches_torch(device, dtype, vocab, hidden, tokens) -> None:
    """Gather == F.embedding; backward == fp64 scatter-add rounded to dtype, then + the tied grad."""
    g = torch.Generator(device=device).manual_seed(vocab + tokens)
    table = torch.randn(vocab, hidden, device=device, generator=g).to(dtype)
    ids = torch.randint(0, vocab, (tokens,), device=device, generator=g)
    ids[:7] = ids[0]  # repeated ids
    ids[7] = vocab - 1
    out = Fn.embedding(table, ids)
    assert torch.equal(out, torch.nn.functional.embedding(ids, table))
    dout = torch.randn(tokens, hidden, device=device, generator=g).to(dtype)
    lm = torch.randn(vocab, hidden, device=device, generator=g).to(dtype)
    sums = torch.zeros(vocab, hidden, dtype=torch.float64, device=device).index_add_(0, ids, dout.double())
    for grad_in in (None, lm):
        grad = torch.empty_like(table)
        Fn._lib.call("nmb_embedding_bwd", dout.data_ptr(), ids.data_ptr(), Fn._lib.ptr(grad_in), grad.data_ptr(),
                     tokens, vocab, hidden, Fn._lib.dtype_code(dtype), Fn._lib.stream_of(dout))
        exp = sums.to(dtype).float() + (grad_in.float() if grad_in is not None else 0.0)
        tol = dict(rtol=1e-2, atol=2e-2) if dtype == torch.bfloat16 else dict(rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(grad.float(), exp.to(dtype).float(), **tol)
        again = torch.empty_like(table)
        Fn._lib.call("nmb_embedding_bwd", dout.data_ptr(), ids.data_ptr(), Fn._lib.ptr(grad_in), again.data_ptr(),
                     tokens, vocab, hidden, Fn._lib.dtype_code(dtype), Fn._lib.stream_of(dout))
        assert torch.equal(grad, again)  # deterministic


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_embedding_backward_hot_row_in_token_order(device, dtype) -> None:
    """One id taking 12,000 of 20,000 tokens (its 16-row block lists more
    tokens than one pass holds, so the rows are added in several batches):
    that row equals the fp32 sum of its gradient rows taken one after another
    in token order (numpy's sequential accumulate), rounded to the dtype, bit
    for bit; every other row is the fp64 scatter-add within the dtype's bar."""
    vocab, hidden, tokens, hot = 512, 256, 20000, 5
    g = torch.Generator(device=device).manual_seed(41)
    ids = torch.randint(0, vocab, (tokens,), device=device, generator=g)
    ids[:12000] = hot
    dout = torch.randn(tokens, hidden, device=device, generator=g).to(dtype)
    grad = torch.empty(vocab, hidden, device=device, dtype=dtype)
    Fn._lib.call("nmb_embedding_bwd", dout.data_ptr(), ids.data_ptr(), None, grad.data_ptr(),
                 tokens, vocab, hidden, Fn._lib.dtype_code(dtype), Fn._lib.stream_of(dout))
    rows = dout[ids == hot].float().cpu().numpy()
    seq = np.add.accumulate(rows, axis=0, dtype=np.float32)[-1]
    assert torch.equal(grad[hot].cpu(), torch.from_numpy(seq).to(dtype))
    sums = torch.zeros(vocab, hidden, dtype=torch.float64, device=device).index_add_(0, ids, dout.double())
    tol = dict(rtol=1e-2, atol=2e-2) if dtype == torch.bfloat16 else dict(rtol=1e-5, atol=1e-5)
    keep = torch.arange(vocab, device=device) != hot
    torch.testing.assert_close(grad[keep].float(), sums[keep].to(dtype).float(), **tol)


@pytest.mark.gpu
def test_tied_embedding_gradient_merge(device) -> None:
    """Embedding + tied LM head in one graph: the merged table gradient equals
    the sum of the two separate gradients."""
    g = torch.Generator(device=device).manual_seed(5)
    bf = torch.bfloat16
    vocab, hidden, b, s = 512, 256, 2, 64
    w = (0.05 * torch.randn(vocab, hidden, device=device, generator=g)).to(bf).requires_grad_()
    ids = torch.randint(0, vocab, (b, s), device=device, generator=g)
    tgt = torch.randint(0, vocab, (b, s), device=device, generator=g)
    tie = Fn.TiedGrad()
    h = Fn.embedding(w, ids, tie)
    loss = Fn.lm_head_cross_entropy(h * 1.5, w, tgt, tie=tie)
    loss.backward()
    merged = w.grad.clone()
    w.grad = None
    h = Fn.embedding(w, ids)
    loss = Fn.lm_head_cross_entropy(h * 1.5, w, tgt)
    loss.backward()  # autograd adds the two gradients
    assert torch.equal(merged, w.grad)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_embedding_out_of_range_ids_match_oracle(device, dtype) -> None:
    """Ids outside [0, V) (negative, V, far beyond V, the ignore value -100) give
    zero rows and no table gradient, as the reference's TP=1 lookup masks them
    (tensor_parallel/embedding.py:63-68): output and table gradient bit-equal to
    the oracle.  The in-range ids are distinct, so every table-gradient row is
    one token's row (or zero) and no summation order enters."""
    g = torch.Generator().manual_seed(9)
    vocab, hidden, b, s = 1000, 256, 4, 64
    table = torch.randn(vocab, hidden, generator=g).to(dtype)
    ids = torch.randperm(vocab, generator=g)[: b * s].view(b, s).clone()
    ids[0, :4] = torch.tensor([-1, vocab, vocab + 5, -100])
    ids[2, 10] = 2**40
    ids[3, 63] = -(2**40)
    dout = torch.randn(b, s, hidden, generator=g).to(dtype)
    wr = table.clone().requires_grad_(True)
    ref = R.embedding_lookup(ids, wr)
    ref.backward(dout)
    wd = table.to(device).requires_grad_(True)
    out = Fn.embedding(wd, ids.to(device))
    out.backward(dout.to(device))
    assert torch.equal(out.cpu(), ref)
    assert not bool(out[0, :4].any()) and not bool(out[2, 10].any())
    assert torch.equal(wd.grad.cpu(), wr.grad)


@pytest.mark.gpu
def test_ring_share_c5_full_size_sampled_rows(device) -> None:
    """Config 5 at full size: rank 3 of a 4-way ring, local queries 24576..32767
    ([1, 8192, 16, 128] bf16) over four 8192-key blocks visited 3, 2, 1, 0
    (context_parallel/ring.py:104-250).  The kernel runs the whole share; the
    oracle checks windows of query rows of two heads (o, lse and dq of a row
    depend on that row alone, over all 32768 keys) and, for one head, dk / dv of
    key windows in the diagonal and a fully visible block (a key's gradient sums
    over every query: the oracle forward over all queries supplies their lse)."""
    s, h, d, nb, rank = 8192, 16, 128, 4, 3
    g = gen(41)
    q = torch.randn(1, s, h, d, generator=g).bfloat16()
    ks = [torch.randn(1, s, h, d, generator=g).bfloat16() for _ in range(nb)]
    vs = [torch.randn(1, s, h, d, generator=g).bfloat16() for _ in range(nb)]
    do = torch.randn(1, s, h, d, generator=g).bfloat16()
    order = [(rank - step) % nb for step in range(nb)]
    offs = [r * s for r in order]
    q_off = rank * s
    kb, vb = [ks[r] for r in order], [vs[r] for r in order]
    qd = q.to(device)
    kbd, vbd = [t.to(device) for t in kb], [t.to(device) for t in vb]
    o, lse = Fn.attn_fwd_bshd(qd, kbd, vbd, offs, causal=True, q_offset=q_off, scale=None)
    dq = torch.empty_like(qd)
    dks = [torch.empty_like(t) for t in kbd]
    dvs = [torch.empty_like(t) for t in vbd]
    Fn.attn_bwd_bshd(qd, kbd, vbd, offs, o, do.to(device), lse, dq, dks, dvs, causal=True,
                     q_offset=q_off, scale=None)
    torch.cuda.synchronize()
    o, lse, dq = o.cpu(), lse.cpu(), dq.cpu()
    dks, dvs = [t.cpu() for t in dks], [t.cpu() for t in dvs]

    def bhsd(t, heads, rows=slice(None)):
        return t[:, rows][:, :, heads].transpose(1, 2).contiguous()

    heads = [0, 9]
    bf = torch.bfloat16
    for start, n in ((0, 48), (4000, 32), (s - 40, 40)):
        rows = slice(start, start + n)
        qr = bhsd(q, heads, rows)
        blocks = [(bhsd(k, heads), bhsd(v, heads)) for k, v in zip(kb, vb)]
        out_ref, lse_ref = R.ring_attention_forward(qr, blocks, offs, causal=True, query_offset=q_off + start)
        dq_ref, _, _ = R.ring_attention_backward(bhsd(do, heads, rows), qr, blocks, offs, out_ref, lse_ref,
                                                 causal=True, query_offset=q_off + start)
        close(bhsd(o, heads, rows), out_ref, bf, msg=f"o rows {start}")
        torch.testing.assert_close(lse[:, heads, rows], lse_ref.squeeze(-1), rtol=1e-3, atol=2e-3)
        close(bhsd(dq, heads, rows), dq_ref, bf, scale_atol=True, msg=f"dq rows {start}")

    head = [9]
    qh = bhsd(q, head)
    blocks = [(bhsd(k, head), bhsd(v, head)) for k, v in zip(kb, vb)]
    out_all, lse_all = R.ring_attention_forward(qh, blocks, offs, causal=True, query_offset=q_off)
    do_h = bhsd(do, head)
    # block index 0 in ring order is the diagonal block (key positions 24576..), 2 is fully visible
    for bi, kstart, n in ((0, 0, 64), (0, s - 64, 64), (2, 1000, 64)):
        keys = slice(kstart, kstart + n)
        kv = [(bhsd(kb[bi], head, keys), bhsd(vb[bi], head, keys))]
        _, dk_ref, dv_ref = R.ring_attention_backward(do_h, qh, kv, [offs[bi] + kstart], out_all, lse_all,
                                                      causal=True, query_offset=q_off)
        close(bhsd(dks[bi], head, keys), dk_ref[0], bf, scale_atol=True, msg=f"dk block {bi} keys {kstart}")
        close(bhsd(dvs[bi], head, keys), dv_ref[0], bf, scale_atol=True, msg=f"dv block {bi} keys {kstart}")


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k,layout", [
    (512, 256, 256, "NT"), (333, 130, 77, "NN"), (65, 1000, 513, "TN"), (128, 64, 8192, "TT"), (1, 7, 3, "NT"),
])
def test_gemm_f32_matches_fp64_product(device, m, n, k, layout) -> None:
    """nmb_gemm_f32 (fp32 MFMA) for every operand layout, ragged tiles, alpha,
    beta and an aliased C, against the fp64 product at the fp32 parity
    tolerance (rtol 1e-5)."""
    g = torch.Generator(device=device).manual_seed(m * 3 + n + k)
    a = torch.randn(m, k, device=device, generator=g) if layout[0] == "N" else torch.randn(k, m, device=device, generator=g).t()
    b = torch.randn(k, n, device=device, generator=g) if layout[1] == "N" else torch.randn(n, k, device=device, generator=g).t()
    c = torch.randn(m, n, device=device, generator=g)
    exp = 0.75 * (a.double() @ b.double()) + 1.5 * c.double()
    out = Fn.mm(a, b, c=c, alpha=0.75, beta=1.5)
    scale = float((a.double().abs() @ b.double().abs()).max())
    torch.testing.assert_close(out.double(), exp, rtol=1e-5, atol=1e-6 * scale)
    acc = c.clone()
    Fn.mm(a, b, out=acc, c=acc, beta=1.0)  # the in-place accumulation the LM head uses
    torch.testing.assert_close(acc.double(), a.double() @ b.double() + c.double(), rtol=1e-5, atol=1e-6 * scale)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_backend_linear_matches_torch_linear(device, dtype) -> None:
    """HipKernelBackend.linear: the nn.Linear parameters and seeded init, with
    the product and its gradients on this library's GEMMs."""
    from nano_megatron_amd.kernels import HipKernelBackend

    torch.manual_seed(3)
    ours = HipKernelBackend().linear(256, 384, bias=False).to(device=device, dtype=dtype)
    torch.manual_seed(3)
    ref = torch.nn.Linear(256, 384, bias=False).to(dtype=dtype)
    assert torch.equal(ours.weight.detach().cpu(), ref.weight.detach())
    g = gen(4)
    x = torch.randn(2, 100, 256, generator=g).to(dtype)
    dy = torch.randn(2, 100, 384, generator=g).to(dtype)
    xr = x.clone().requires_grad_(True)
    yr = ref(xr)
    yr.backward(dy)
    xd = x.to(device).requires_grad_(True)
    yd = ours(xd)
    yd.backward(dy.to(device))
    close(yd, yr, dtype)
    close(xd.grad, xr.grad, dtype, scale_atol=True)
    close(ours.weight.grad, ref.weight.grad, dtype, scale_atol=True)


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k,at,bt", [(8192, 1024, 2048, True, True), (1024, 1024, 8192, True, True),
                                         (304, 520, 136, False, False), (2048, 3072, 1024, False, True)])
def test_gemm_f32out_is_the_bf16_gemm_before_its_rounding(device, m, n, k, at, bt) -> None:
    """nmb_gemm_bf16_f32out (beta 0) rounded to bf16 equals nmb_gemm_bf16 bit for
    bit (same plan and sums, split along K or not); its fp32 values lie within
    the fp32 summation bound of the exact product; alpha and beta apply in fp32."""
    g = torch.Generator(device=device).manual_seed(m + n + k)
    bf = torch.bfloat16
    a = torch.randn(k, m, device=device, generator=g).to(bf).t() if at else \
        torch.randn(m, k, device=device, generator=g).to(bf)
    b = torch.randn(k, n, device=device, generator=g).to(bf) if bt else \
        torch.randn(n, k, device=device, generator=g).to(bf).t()
    out = torch.empty(m, n, dtype=torch.float32, device=device)
    Fn.mm_f32out(a, b, out)
    assert torch.equal(out.to(bf), Fn.mm(a, b))
    exact = a.double() @ b.double()
    bound = k * 2.0 ** -24 * (a.double().abs() @ b.double().abs())
    assert bool(((out.double() - exact).abs() <= bound).all())
    twice = out.clone()
    Fn.mm_f32out(a, b, twice, beta=1.0)
    assert torch.equal(twice, 2 * out)
    half = torch.empty_like(out)
    Fn.mm_f32out(a, b, half, alpha=0.5)
    assert torch.equal(half, 0.5 * out)


@pytest.mark.gpu
def test_lm_head_table_gradient_is_rounded_once(device) -> None:
    """The tied LM head's table gradient, accumulated over four 2048-token chunks,
    is the bf16 rounding of a value within the fp32 summation bound of the exact
    sum of G_c^T x_c (as the reference's single product G^T X is rounded once),
    not the sum of four rounded chunk products."""
    g = torch.Generator(device=device).manual_seed(11)
    bf = torch.bfloat16
    t, h, v, chunk = 8192, 1024, 8192, 2048
    x = torch.randn(t, h, device=device, generator=g).to(bf)
    w = (0.02 * torch.randn(v, h, device=device, generator=g)).to(bf).requires_grad_()
    y = torch.randint(0, v, (t,), device=device, generator=g)
    Fn.lm_head_cross_entropy(x, w, y, reduction="sum", chunk=chunk).backward()
    # the chunks' G exactly as the backward forms them (same kernels, same inputs)
    with torch.no_grad():
        loss = torch.empty(t, dtype=torch.float32, device=device)
        lse = torch.empty_like(loss)
        ones = torch.ones(t, dtype=torch.float32, device=device)
        exact = torch.zeros(v, h, dtype=torch.float64, device=device)
        absum = torch.zeros_like(exact)
        for s in range(0, t, chunk):
            logits = Fn.mm(x[s:s + chunk], w.detach().t())
            Fn.ce_fwd(logits, y[s:s + chunk], -100, loss[s:s + chunk], lse[s:s + chunk])
            Fn.ce_bwd_(logits, y[s:s + chunk], -100, lse[s:s + chunk], ones[s:s + chunk])
            exact += logits.double().t() @ x[s:s + chunk].double()
            absum += logits.double().abs().t() @ x[s:s + chunk].double().abs()
        bound = t * 2.0 ** -24 * absum
        mag = exact.abs() + bound
        half_ulp = torch.where(mag > 0, torch.exp2(torch.floor(torch.log2(mag)) - 8), torch.zeros_like(mag))
        err = (w.grad.double() - exact).abs()
        assert bool((err <= half_ulp + bound).all()), float((err - half_ulp - bound).max())


@pytest.mark.parametrize("n_in,n_out", [(100, 52), (96, 1001), (37, 8)])
def test_linear_with_feature_counts_not_multiples_of_8(device, n_in, n_out) -> None:
    """HipKernelBackend.linear for any feature counts (nn.Linear's contract):
    the bf16 GEMM runs on zero-padded copies; forward and both gradients
    against fp32 products."""
    backend = nm.HipKernelBackend()
    torch.manual_seed(n_in + n_out)
    lin = backend.linear(n_in, n_out, bias=True).to(device=device, dtype=torch.bfloat16)
    x = torch.randn(3, 41, n_in, device=device).bfloat16().requires_grad_(True)
    dy = torch.randn(3, 41, n_out, device=device).bfloat16()
    y = lin(x)
    y.backward(dy)
    xf, wf = x.detach().float(), lin.weight.detach().float()
    ref = xf @ wf.t() + lin.bias.detach().float()
    assert y.shape == (3, 41, n_out)
    torch.testing.assert_close(y.float(), ref, rtol=2e-2, atol=2e-2 * float(ref.abs().max()))
    dxr = dy.float() @ wf
    dwr = dy.float().reshape(-1, n_out).t() @ xf.reshape(-1, n_in)
    torch.testing.assert_close(x.grad.float(), dxr, rtol=2e-2, atol=2e-2 * float(dxr.abs().max()))
    torch.testing.assert_close(lin.weight.grad.float(), dwr, rtol=2e-2, atol=2e-2 * float(dwr.abs().max()))


@pytest.mark.parametrize("d,hq,hkv,causal", [(96, 4, 2, True), (32, 2, 2, False), (80, 4, 1, True)])
def test_attention_other_head_sizes_bf16(device, d, hq, hkv, causal) -> None:
    """local_attention at head sizes other than 64 and 128 in bf16 (SDPA takes
    any): the MFMA kernels on zero-padded heads, forward and gradients against
    the oracle."""
    g = gen(d + hq)
    q = torch.randn(2, hq, 70, d, generator=g).bfloat16()
    k = torch.randn(2, hkv, 70, d, generator=g).bfloat16()
    v = torch.randn(2, hkv, 70, d, generator=g).bfloat16()
    do = torch.randn(2, hq, 70, d, generator=g).bfloat16()
    qr, kr, vr = (t.float().clone().requires_grad_(True) for t in (q, k, v))
    o_ref = R.local_attention(qr, kr, vr, causal=causal)
    o_ref.backward(do.float())
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    o = nm.HipKernelBackend().local_attention(qd, kd, vd, causal=causal)
    o.backward(do.to(device))
    close(o, o_ref, torch.bfloat16)
    close(qd.grad, qr.grad, torch.bfloat16, scale_atol=True, msg="dq")
    close(kd.grad, kr.grad, torch.bfloat16, scale_atol=True, msg="dk")
    close(vd.grad, vr.grad, torch.bfloat16, scale_atol=True, msg="dv")


def test_rmsnorm_bwd_dw_on_a_second_stream_is_bit_identical(device) -> None:
    """nmb_rmsnorm_bwd_rows + nmb_rmsnorm_bwd_dw with the column sum on another
    stream (as the block backward runs the post-attention norm) equal
    nmb_rmsnorm_bwd bit for bit."""
    g = torch.Generator(device=device).manual_seed(3)
    x = torch.randn(8192, 1024, device=device, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(1024, device=device, generator=g)).bfloat16()
    dy = torch.randn(8192, 1024, device=device, generator=g).bfloat16()
    res = torch.randn(8192, 1024, device=device, generator=g).bfloat16()
    side = torch.cuda.Stream(device)
    dx0, dw0 = Fn.rmsnorm_bwd(x, w, dy, 1e-5, residual_grad=res)
    dx1, dw1 = Fn.rmsnorm_bwd(x, w, dy, 1e-5, residual_grad=res, dw_stream=side)
    torch.cuda.current_stream(device).wait_stream(side)
    assert torch.equal(dx0, dx1) and torch.equal(dw0, dw1)


# the config shapes, odd K-tile counts (136, 264: the second product loads its
# own first tiles), two K tiles (128: both preloaded) and one (64)
@pytest.mark.parametrize("m,f,h", [(8192, 2736, 1024), (8192, 5632, 2048), (300, 200, 136), (512, 136, 264),
                                   (256, 136, 128), (300, 72, 64)])
def test_gate_up_swiglu_bwd_equals_gate_up_then_swiglu_bwd(device, m, f, h) -> None:
    """nmb_gemm_bf16_gate_up_swiglu_bwd (the recomputed gate/up product, ds =
    dY Wd and the SwiGLU backward in one kernel, [g|u] never in memory) equals
    the gate/up product followed by nmb_gemm_bf16_swiglu_bwd bit for bit, at
    the config-3 and config-4 shapes and ragged ones (partial row and F tiles)."""
    g = torch.Generator(device=device).manual_seed(m + f + h)
    bf = torch.bfloat16
    n2 = torch.randn(m, h, device=device, generator=g).to(bf)
    wgu = (0.05 * torch.randn(2 * f, h, device=device, generator=g)).to(bf)
    dy = torch.randn(m, h, device=device, generator=g).to(bf)
    wd = (0.05 * torch.randn(h, f, device=device, generator=g)).to(bf)
    _, gu = Fn.mm_gate_up(n2, wgu, act=False, gu=True)
    dgu_ref, act_ref = Fn.mm_swiglu_bwd(dy, wd, gu)
    dgu, act = Fn.mm_gate_up_swiglu_bwd(n2, wgu, dy, wd)
    assert torch.equal(dgu, dgu_ref)
    assert torch.equal(act, act_ref)
    dgu2, none = Fn.mm_gate_up_swiglu_bwd(n2, wgu, dy, wd, act=False)
    assert none is None and torch.equal(dgu2, dgu)
