"""Dropout on the GPU: the residual-add dropout kernel and attention dropout
against the oracle on the same keep masks (bit for bit where the arithmetic
is elementwise, fp32 rtol 1e-5 / bf16 rtol 2e-2 elsewhere), torch's own GPU
dropout arithmetic against the oracle's, and the model with dropout against
the oracle model given the same mask keys.  The reference draws its masks from
torch's Philox stream, which no other generator reproduces; parity is on the
arithmetic and placement of dropout for a given mask, and on the mask's
statistics."""

from __future__ import annotations

import hashlib
import math
from contextlib import contextmanager

import pytest
import torch

import nano_megatron_amd as nm
from nano_megatron_amd import _lib
from nano_megatron_amd import functional as Fn
from nano_megatron_amd.graph import CapturedTrainStep
from nano_megatron_amd.optim import MasterAdamW
from oracle import reference as R
from parity import assert_bf16_grads, assert_close_scaled, assert_grads_scaled, assert_loss_close

pytestmark = pytest.mark.gpu


def gen(seed):
    return torch.Generator().manual_seed(seed)


def close(got, exp, dtype, scale_atol=True, msg=""):
    """The dtype's bar with atol scaled to max|exp| (tests/parity.py)."""
    assert_close_scaled(got, exp, dtype, msg=msg)


# ---------------------------------------------------------------- elementwise dropout
@pytest.mark.parametrize("p", [0.1, 0.37])
def test_torch_gpu_dropout_rounds_as_the_oracle(device, p) -> None:
    """The reference's F.dropout on the GPU (native_dropout also returns its
    mask) rounds x / (1 - p) in fp32 to bf16: the oracle's arithmetic with
    torch's mask gives torch's output bit for bit."""
    x = torch.randn(1 << 16, generator=gen(1)).bfloat16().to(device)
    out, mask = torch.ops.aten.native_dropout(x, p, True)
    assert torch.equal(R.dropout_apply(x.cpu(), mask.cpu(), p), out.cpu())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,offset,residual", [
    (16 * 512 * 1024, 0, True),   # config 3's [B*S, H]
    (16 * 512 * 1024, 0, False),
    (1001, 0, True),              # ragged: the vector path and a scalar tail
    (999, 1, True),               # misaligned by one element: all scalar
    (7, 0, False),
    (0, 0, True),
])
def test_dropout_add_matches_oracle(device, dtype, n, offset, residual) -> None:
    p, seed = 0.1, 0x1234_5678_9ABC
    g = gen(2)
    # slice on the device, so that offset 1 really misaligns the pointers
    xd = torch.randn(n + offset, generator=g).to(dtype).to(device)[offset:]
    rd = torch.randn(n + offset, generator=g).to(dtype).to(device)[offset:] if residual else None
    got = Fn.dropout_add(xd, p, seed=seed, residual=rd)
    exp = R.dropout_add(xd.cpu(), p, seed, residual=None if rd is None else rd.cpu())
    assert torch.equal(got.cpu(), exp)
    if n >= 1 << 20:
        kept = float((R.dropout_keep(seed, (n,), p)).float().mean())
        assert abs(kept - (1 - p)) < 5 * math.sqrt(p * (1 - p) / n)


def test_dropout_add_backward_and_determinism(device) -> None:
    """d x = dropout(d out) with the same mask, d residual = d out; the same
    seed gives the same output, another seed another mask; p = 0 is exact."""
    g = gen(3)
    x = torch.randn(64, 1024, generator=g).bfloat16().to(device).requires_grad_(True)
    r = torch.randn(64, 1024, generator=g).bfloat16().to(device).requires_grad_(True)
    dy = torch.randn(64, 1024, generator=g).bfloat16().to(device)
    y = Fn.dropout_add(x, 0.2, seed=77, residual=r)
    y.backward(dy)
    assert torch.equal(x.grad.cpu(), R.dropout_add(dy.cpu(), 0.2, 77))
    assert torch.equal(r.grad, dy)
    assert torch.equal(Fn.dropout_add(x.detach(), 0.2, seed=77, residual=r.detach()), y.detach())
    assert not torch.equal(Fn.dropout_add(x.detach(), 0.2, seed=78, residual=r.detach()), y.detach())
    assert torch.equal(Fn.dropout_add(x.detach(), 0.0, seed=5), x.detach())


def test_dropout_add_in_place_through_the_abi(device) -> None:
    """out may alias x (the header allows it): the in-place call equals the
    out-of-place one."""
    x = torch.randn(4099, generator=gen(4)).bfloat16().to(device)
    r = torch.randn(4099, generator=gen(5)).bfloat16().to(device)
    exp = Fn.dropout_add(x, 0.3, seed=9, residual=r)
    y = x.clone()
    _lib.call("nmb_dropout_add", y.data_ptr(), r.data_ptr(), y.data_ptr(), y.numel(), 0.3, 9,
              _lib.NMB_BF16, _lib.stream_of(y))
    assert torch.equal(y, exp)


# ---------------------------------------------------------------- attention dropout
ATTN_DROP_CASES = [
    # (dtype, causal, offset, mask, hq, hkv, sq, sk, d, p)
    (torch.float32, True, 0, None, 4, 2, 48, 48, 64, 0.2),
    (torch.float32, False, 0, "add", 2, 1, 29, 31, 80, 0.35),
    (torch.bfloat16, True, 0, None, 4, 4, 64, 64, 64, 0.1),
    (torch.bfloat16, True, 5, "bool", 8, 2, 37, 45, 128, 0.25),
]


@pytest.mark.parametrize("dtype,causal,offset,mask_kind,hq,hkv,sq,sk,d,p", ATTN_DROP_CASES)
def test_attention_dropout_matches_oracle(device, dtype, causal, offset, mask_kind, hq, hkv, sq, sk, d,
                                          p) -> None:
    """local_attention(dropout_p=p) through the HIP backend against the oracle
    (torch's math SDPA given the same keep mask): forward and q/k/v gradients,
    with and without a mask, GQA, offsets, ragged lengths."""
    g = gen(8)
    b, seed = 2, 4242
    q = torch.randn(b, hq, sq, d, generator=g).to(dtype)
    k = torch.randn(b, hkv, sk, d, generator=g).to(dtype)
    v = torch.randn(b, hkv, sk, d, generator=g).to(dtype)
    do = torch.randn(b, hq, sq, d, generator=g).to(dtype)
    mask = None
    if mask_kind == "bool":
        mask = torch.rand(b, 1, sq, sk, generator=g) > 0.3
    elif mask_kind == "add":
        mask = torch.randn(sq, sk, generator=g).to(dtype)
    qr, kr, vr = (t.float().clone().requires_grad_(True) for t in (q, k, v))
    mr = None if mask is None else (mask if mask.dtype == torch.bool else mask.float())
    o_ref = R.local_attention(qr, kr, vr, causal=causal, sequence_offset=offset, attention_mask=mr,
                              dropout_p=p, dropout_seed=seed)
    o_ref.backward(do.float())
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    o = Fn.masked_attention(qd, kd, vd, None if mask is None else mask.to(device), causal=causal,
                            sequence_offset=offset, dropout_p=p, seed=seed)
    o.backward(do.to(device))
    close(o, o_ref, dtype)
    close(qd.grad, qr.grad, dtype, scale_atol=True, msg="dq")
    close(kd.grad, kr.grad, dtype, scale_atol=True, msg="dk")
    close(vd.grad, vr.grad, dtype, scale_atol=True, msg="dv")


def test_attention_dropout_through_the_seam_replays_the_generator(device) -> None:
    """The backend draws the mask key from torch's default CPU generator: the
    same generator state gives the same output, and dropout_p = 0 equals the
    plain attention."""
    g = gen(9)
    q, k, v = (torch.randn(1, 4, 32, 64, generator=g).bfloat16().to(device) for _ in range(3))
    backend = nm.HipKernelBackend()
    torch.manual_seed(17)
    a = backend.local_attention(q, k, v, dropout_p=0.3)
    torch.manual_seed(17)
    b = backend.local_attention(q, k, v, dropout_p=0.3)
    c = backend.local_attention(q, k, v, dropout_p=0.3)
    assert torch.equal(a, b) and not torch.equal(a, c)
    assert torch.equal(backend.local_attention(q, k, v, dropout_p=0.0), nm.attention(q, k, v))


# ---------------------------------------------------------------- model
class ForkRNG:
    """A stream tracker with the reference's fork() interface (parallel/rng.py:
    111-131): reseeds torch's default CPU generator with a stable hash of the
    components for the duration of the block."""

    def __init__(self, base: int) -> None:
        self.base = base
        self.forks = 0

    def seed_of(self, components) -> int:
        text = "|".join(str(c) for c in (self.base, *components)).encode()
        return int.from_bytes(hashlib.blake2b(text, digest_size=8).digest(), "little") % (2**63 - 1)

    @contextmanager
    def fork(self, stream, *, components=(), cuda_devices=None, advance=True):
        self.forks += 1
        with torch.random.fork_rng(devices=[]):
            torch.random.default_generator.manual_seed(self.seed_of(components))
            yield


def kernel_seed(fork_seed: int) -> int:
    """The key functional.dropout_seed() draws right after the fork reseeds."""
    g = torch.Generator().manual_seed(fork_seed)
    return int(torch.randint(0, 2**63 - 1, (1,), dtype=torch.int64, generator=g).item())


def model_pair(device, dtype, mode, rng, kv_heads=None, dropout=0.1):
    cfg = nm.GPTConfig(layers=2, hidden_size=256, ffn_hidden_size=688, heads=4, kv_heads=kv_heads,
                       seq_length=64, vocab_size=4096, norm_epsilon=1e-5, dropout=dropout)
    ck = nm.ActivationCheckpointConfig(mode=mode)
    torch.manual_seed(0)
    ours = nm.GPTModel(cfg, activation_checkpoint_config=ck, rng=rng).to(device=device, dtype=dtype)
    seeds = (lambda layer, op: kernel_seed(rng.seed_of((layer, 0, 0, op)))) if rng is not None else None
    ref = R.OracleGPTModel(cfg, activation_checkpoint_config=ck, dropout_seed=seeds).to(dtype=dtype)
    ref.load_state_dict({k: v.cpu() for k, v in ours.state_dict().items()})
    ours.train()
    ref.train()
    return ours, ref


def fp32_twin(ref, rng):
    """The oracle in fp32 on the bf16 oracle's weights, with the same masks."""
    seeds = (lambda layer, op: kernel_seed(rng.seed_of((layer, 0, 0, op)))) if rng is not None else None
    twin = R.OracleGPTModel(ref.config, activation_checkpoint_config=ref.activation_checkpoint_config,
                            dropout_seed=seeds)
    twin.load_state_dict({k: v.float() for k, v in ref.state_dict().items()})
    return twin.train()


def batch():
    ids = torch.randint(0, 4096, (2, 65), generator=gen(10))
    return ids[:, :64].contiguous(), ids[:, 1:].contiguous()


@pytest.mark.parametrize("dtype,mode,kv_heads", [
    (torch.float32, "full", None), (torch.float32, "none", 2), (torch.bfloat16, "full", 2),
    (torch.bfloat16, "selective", None),
])
def test_model_with_dropout_matches_oracle(device, dtype, mode, kv_heads) -> None:
    """Embedding, attention and both residual dropouts at p = 0.1 with masks
    keyed by (layer, microbatch, offset, op) through the rng's fork: loss and
    every gradient against the oracle model given the same keys."""
    rng = ForkRNG(1234)
    ours, ref = model_pair(device, dtype, mode, rng, kv_heads)
    ids, labels = batch()
    lo = ours(ids.to(device), labels=labels.to(device)).loss
    lr = ref(ids, labels=labels).loss
    lo.backward()
    lr.backward()
    assert_loss_close(lo, lr, dtype)
    if dtype == torch.float32:
        assert_grads_scaled(ours, ref, dtype)
    else:
        twin = fp32_twin(ref, rng)
        twin(ids, labels=labels).loss.backward()
        assert_bf16_grads(ours, ref, twin)
    assert rng.forks > 0


@pytest.mark.parametrize("use_rng", [False, True])
def test_dropout_recompute_replays_the_masks(device, use_rng) -> None:
    """Full recompute with dropout: the checkpoint's recompute regenerates the
    forward's masks (torch's checkpoint replays the CPU generator; a forked
    stream is keyed by position), so loss and gradients equal the
    no-checkpoint run bit for bit."""
    ids, labels = batch()
    grads = []
    for mode in ("full", "none"):
        ours, _ = model_pair(device, torch.bfloat16, mode, ForkRNG(7) if use_rng else None)
        torch.manual_seed(99)
        loss = ours(ids.to(device), labels=labels.to(device)).loss
        loss.backward()
        grads.append((loss.detach(), [p.grad.clone() for p in ours.parameters()]))
    assert torch.equal(grads[0][0], grads[1][0])
    for a, b in zip(grads[0][1], grads[1][1]):
        assert torch.equal(a, b)


def test_dropout_is_off_in_eval_and_refused_by_graph_capture(device) -> None:
    ours, ref = model_pair(device, torch.float32, "full", ForkRNG(3))
    ours.eval()
    ref.eval()
    ids, labels = batch()
    with torch.no_grad():
        lo = ours(ids.to(device), labels=labels.to(device)).loss
        lr = ref(ids, labels=labels).loss
    torch.testing.assert_close(lo.cpu(), lr, rtol=1e-5, atol=1e-5)
    ours.train()
    opt = MasterAdamW(ours.parameters(), lr=1e-4)
    with pytest.raises(ValueError, match="dropout"):
        CapturedTrainStep(ours, opt, ids.to(device), labels.to(device))
