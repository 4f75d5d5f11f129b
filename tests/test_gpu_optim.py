"""Fused fp32-master AdamW + global grad-norm clip (nmb_adamw_step) against the
oracle's FlatShardZeROStrategy arithmetic (data_parallel/_zero.py:130-199)."""

from __future__ import annotations

import pytest
import torch

from nano_megatron_amd.optim import MasterAdamW
from oracle import reference as R

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,max_norm", [(torch.bfloat16, 1.0), (torch.float32, 1.0),
                                            (torch.bfloat16, None)])
def test_master_adamw_matches_oracle(device, dtype, max_norm) -> None:
    g = torch.Generator().manual_seed(3)
    shapes = [(1024,), (300, 7), (64, 1024), (5,), (40000,)]
    init = [torch.randn(*s, generator=g) * 0.1 for s in shapes]
    params = [torch.nn.Parameter(t.to(dtype).to(device)) for t in init]
    opt = MasterAdamW(params, lr=1e-3, weight_decay=0.1, clip_grad_norm=max_norm)
    master = [t.to(dtype).float() for t in init]
    m = [torch.zeros_like(t) for t in master]
    v = [torch.zeros_like(t) for t in master]
    for step in range(1, 4):
        grads = [(torch.randn(*s, generator=g) * (3.0 if step == 2 else 0.01)).to(dtype) for s in shapes]
        for p, gr in zip(params, grads):
            p.grad = gr.to(device)
        opt.step()
        gf = [gr.float() for gr in grads]
        norm = torch.sqrt(sum((x * x).sum() for x in gf))
        coef = R.clip_coefficient(norm, max_norm) if max_norm else torch.tensor(1.0)
        for w, mm, vv, gg in zip(master, m, v, gf):
            R.adamw_master_step(w, mm, vv, gg * coef, step=step, lr=1e-3, weight_decay=0.1)
        torch.testing.assert_close(opt.last_grad_norm.cpu(), norm, rtol=1e-5, atol=1e-6)
        got = opt.master.cpu()
        exp = torch.cat([w.reshape(-1) for w in master])
        torch.testing.assert_close(got, exp, rtol=1e-5, atol=1e-6)
        off = 0
        for p in params:
            n = p.numel()
            mine = got[off:off + n].view_as(p).to(dtype)
            assert torch.equal(p.detach().cpu(), mine), "parameter != cast(master)"
            off += n


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_master_adamw_moments_are_bit_exact(device, dtype) -> None:
    """Without clipping (coefficient exactly 1) the moments follow the oracle's
    torch operations bit for bit (m.mul_(b1).add_(g, alpha), v.mul_(b2).addcmul_),
    and the master stays within an ulp of itself plus an ulp of the update's
    scale per step (torch's CPU square root is not always correctly rounded;
    the kernel's is; where w and the update nearly cancel, the update's ulp
    dominates)."""
    g = torch.Generator().manual_seed(7)
    shapes = [(4096,), (33, 17), (100000,)]
    init = [torch.randn(*s, generator=g) * 0.1 for s in shapes]
    params = [torch.nn.Parameter(t.to(dtype).to(device)) for t in init]
    opt = MasterAdamW(params, lr=1e-3, weight_decay=0.1, clip_grad_norm=None)
    master = [t.to(dtype).float() for t in init]
    m = [torch.zeros_like(t) for t in master]
    v = [torch.zeros_like(t) for t in master]
    cat = lambda xs: torch.cat([x.reshape(-1) for x in xs])  # noqa: E731
    for step in range(1, 5):
        grads = [(torch.randn(*s, generator=g) * 0.01).to(dtype) for s in shapes]
        for p, gr in zip(params, grads):
            p.grad = gr.to(device)
        opt.step()
        for w, mm, vv, gr in zip(master, m, v, grads):
            R.adamw_master_step(w, mm, vv, gr.float(), step=step, lr=1e-3, weight_decay=0.1)
        assert torch.equal(opt.exp_avg.cpu(), cat(m))
        assert torch.equal(opt.exp_avg_sq.cpu(), cat(v))
        got, exp = opt.master.cpu(), cat(master)
        ulp = torch.nextafter(exp.abs(), torch.tensor(float("inf"))) - exp.abs()
        update_ulp = torch.nextafter(torch.tensor(10 * 1e-3), torch.tensor(1.0)) - torch.tensor(10 * 1e-3)
        assert bool(((got - exp).abs() <= step * (ulp + update_ulp)).all())
        assert (got != exp).float().mean().item() < 5e-2
