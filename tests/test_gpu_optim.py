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
