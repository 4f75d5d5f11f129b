"""fp32-master AdamW with global gradient-norm clipping on ``nmb_adamw_step``.

Mirrors the single-rank arithmetic of FlatShardZeROStrategy
(data_parallel/_zero.py:95-114 master init, :130-164 clip_grad_norm,
:166-199 optimizer_step) with the reference defaults (config/schema.py:439-445):
betas (0.9, 0.95), eps 1e-8, weight decay 0.1, clip 1.0.  The master weights
and both moments are flat fp32 device arrays; one call clips and updates every
parameter and writes the (bf16) parameters back, without a host sync.
"""

from __future__ import annotations

from typing import Iterable

import torch
from torch import Tensor, nn

from nano_megatron_amd import _lib


class MasterAdamW:
    def __init__(self, params: Iterable[nn.Parameter], *, lr: float = 3.0e-4,
                 betas: tuple[float, float] = (0.9, 0.95), eps: float = 1.0e-8,
                 weight_decay: float = 0.1, clip_grad_norm: float | None = 1.0) -> None:
        self.params = [p for p in params if p.requires_grad]
        if not self.params:
            raise ValueError("MasterAdamW needs at least one parameter")
        device = self.params[0].device
        if device.type != "cuda" or any(p.device != device for p in self.params):
            raise ValueError("MasterAdamW runs on one GPU: all parameters must be on the same HIP device")
        if len({p.dtype for p in self.params}) != 1:
            raise ValueError("MasterAdamW needs one parameter dtype")
        self.lr, self.betas, self.eps, self.weight_decay = float(lr), tuple(betas), float(eps), float(weight_decay)
        self.max_norm = float(clip_grad_norm) if clip_grad_norm else 0.0
        self.device = device
        numels = [p.numel() for p in self.params]
        offsets = [0]
        for n in numels:
            offsets.append(offsets[-1] + n)
        self.total = offsets[-1]
        self.offsets = torch.tensor(offsets, dtype=torch.int64, device=device)
        self.master = torch.cat([p.detach().reshape(-1).float() for p in self.params])
        self.exp_avg = torch.zeros_like(self.master)
        self.exp_avg_sq = torch.zeros_like(self.master)
        nbytes = _lib.ctypes.c_size_t(0)
        _lib.call("nmb_adamw_workspace_bytes", self.total, _lib.ctypes.byref(nbytes))
        self.workspace = torch.empty(nbytes.value, dtype=torch.uint8, device=device)
        self.stats = torch.zeros(2, dtype=torch.float32, device=device)  # [norm, coef]
        self.step_count = 0
        self._param_table = torch.tensor([p.data_ptr() for p in self.params], dtype=torch.int64,
                                         device=device)
        self._param_ptrs = [p.data_ptr() for p in self.params]

    @property
    def last_grad_norm(self) -> Tensor:
        return self.stats[0]

    def zero_grad(self, set_to_none: bool = True) -> None:
        for p in self.params:
            if set_to_none:
                p.grad = None
            elif p.grad is not None:
                p.grad.zero_()

    @torch.no_grad()
    def step(self) -> None:
        grads = []
        for p in self.params:
            if p.grad is None:
                raise ValueError("MasterAdamW.step: every parameter needs a gradient")
            g = p.grad
            if not g.is_contiguous() or g.dtype != p.grad.dtype:
                g = g.contiguous()
            grads.append(g)
        gdt = {g.dtype for g in grads}
        if len(gdt) != 1:
            raise ValueError("MasterAdamW.step: gradients must share one dtype")
        ptrs = [p.data_ptr() for p in self.params]
        if ptrs != self._param_ptrs:  # parameters were moved or repacked
            self._param_table = torch.tensor(ptrs, dtype=torch.int64, device=self.device)
            self._param_ptrs = ptrs
        table = torch.tensor([g.data_ptr() for g in grads], dtype=torch.int64).pin_memory()
        grad_table = table.to(self.device, non_blocking=True)
        self.step_count += 1
        _lib.call(
            "nmb_adamw_step", self._param_table.data_ptr(), grad_table.data_ptr(),
            self.offsets.data_ptr(), len(self.params), self.total, self.master.data_ptr(),
            self.exp_avg.data_ptr(), self.exp_avg_sq.data_ptr(),
            _lib.dtype_code(self.params[0].dtype), _lib.dtype_code(gdt.pop()), self.lr,
            self.betas[0], self.betas[1], self.eps, self.weight_decay, self.step_count,
            self.max_norm, self.stats.data_ptr(), self.workspace.data_ptr(), self.workspace.numel(),
            _lib.stream_of(self.master),
        )
        self._keep = (grads, grad_table)  # alive until the next step's kernels are enqueued
