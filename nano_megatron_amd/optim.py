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
        self._graph: dict | None = None  # buffers of a captured step (prepare_graph)

    def set_learning_rate(self, lr: float) -> None:
        """The rate of the next update (a schedule installs it between steps)."""
        if isinstance(lr, bool) or not lr >= 0.0:
            raise ValueError(f"learning rate must be >= 0, got {lr!r}")
        self.lr = float(lr)

    @property
    def last_grad_norm(self) -> Tensor:
        return self.stats[0]

    def state_dict(self) -> dict:
        """This optimizer's own resumable state: the fp32 master, both moments,
        the step count and the rate, as host tensors over the flat layout of
        the parameters (in their order), with their element counts.  It holds
        what the reference's ZeRO strategy saves at one rank
        (data_parallel/_zero.py:234-251) but not in its per-bucket layout:
        neither side loads the other's state."""
        return {
            "mode": "master_adamw",
            "step": self.step_count,
            "learning_rate": self.lr,
            "numels": [p.numel() for p in self.params],
            "master_parameter": self.master.detach().cpu(),
            "exp_avg": self.exp_avg.detach().cpu(),
            "exp_avg_sq": self.exp_avg_sq.detach().cpu(),
        }

    @torch.no_grad()
    def load_state_dict(self, state: dict) -> None:
        """Restores what ``state_dict`` saved; the element counts must match
        the current parameters.  The master, both moments, the step and the
        rate come back (the parameters themselves come from the model's state
        dict)."""
        if state.get("mode", "master_adamw") != "master_adamw":
            raise ValueError(f"cannot load {state.get('mode')!r} state into MasterAdamW")
        numels = [p.numel() for p in self.params]
        if list(state.get("numels", numels)) != numels:
            raise ValueError(f"parameter layout changed: saved={state.get('numels')}, current={numels}")
        for key, target in (("master_parameter", self.master), ("exp_avg", self.exp_avg),
                            ("exp_avg_sq", self.exp_avg_sq)):
            full = state.get(key)
            if not isinstance(full, Tensor) or full.numel() != self.total:
                raise ValueError(f"{key} has an incompatible logical shape")
            target.copy_(full.reshape(-1).to(device=self.device, dtype=torch.float32))
        self.step_count = int(state.get("step", 0))
        self.set_learning_rate(float(state.get("learning_rate", self.lr)))

    def zero_grad(self, set_to_none: bool = True) -> None:
        for p in self.params:
            if set_to_none:
                p.grad = None
            elif p.grad is not None:
                p.grad.zero_()

    def prepare_graph(self) -> None:
        """Buffers a step captured in a HIP graph needs, allocated before the
        capture: a device record of the update's scalars (``advance_graph_step``
        refreshes it before each replay; the launch arguments of a graph are
        fixed) and a pinned staging copy of the gradient pointer table, which
        the captured step copies to the device.  Refreshes the parameter table
        if the parameters moved."""
        ptrs = [p.data_ptr() for p in self.params]
        if ptrs != self._param_ptrs:
            self._param_table = torch.tensor(ptrs, dtype=torch.int64, device=self.device)
            self._param_ptrs = ptrs
        nb = _lib.ctypes.c_size_t(0)
        _lib.call("nmb_adamw_hyper_bytes", _lib.ctypes.byref(nb))
        n = len(self.params)
        self._graph = dict(
            # two host records, alternating: one may still wait for its copy to
            # the device while the next step's scalars are written to the other
            hyper_host=[torch.empty(nb.value, dtype=torch.uint8, pin_memory=True) for _ in range(2)],
            hyper_copied=[None, None],
            hyper_next=0,
            hyper_dev=torch.empty(nb.value, dtype=torch.uint8, device=self.device),
            table_host=torch.empty(n, dtype=torch.int64, pin_memory=True),
            table_dev=torch.empty(n, dtype=torch.int64, device=self.device),
        )

    def advance_graph_step(self) -> None:
        """Before a replay of a captured step: the step count advances as an
        eager ``step`` would advance it, and the update's scalars for that
        step go to the device on the current stream (stream-ordered after the
        previous replay, whose update has read the device record by then).
        The host records alternate; before one is rewritten the host waits for
        the copy that last read it, two steps back, so it never waits for the
        replay in flight."""
        if self._graph is None:
            raise ValueError("MasterAdamW.advance_graph_step: call prepare_graph() before capturing")
        self.step_count += 1
        i = self._graph["hyper_next"]
        self._graph["hyper_next"] = 1 - i
        host = self._graph["hyper_host"][i]
        copied = self._graph["hyper_copied"][i]
        if copied is not None:
            copied.synchronize()
        _lib.call("nmb_adamw_hyper", self.lr, self.betas[0], self.betas[1], self.eps,
                  self.weight_decay, self.step_count, host.data_ptr())
        self._graph["hyper_dev"].copy_(host, non_blocking=True)
        copied = torch.cuda.Event()
        copied.record(torch.cuda.current_stream(self.device))
        self._graph["hyper_copied"][i] = copied

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
        if self.device.type == "cuda" and torch.cuda.is_current_stream_capturing():
            self._captured_step(grads, gdt.pop(), ptrs)
            return
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

    def _captured_step(self, grads: list[Tensor], gdtype: torch.dtype, ptrs: list[int]) -> None:
        """The step as a graph records it: the gradient table is copied from the
        pinned staging buffer (a copy node), the scalars come from the device
        record; the step count advances per replay (``advance_graph_step``)."""
        if self._graph is None:
            raise ValueError("MasterAdamW.step under HIP graph capture needs prepare_graph() first")
        if ptrs != self._param_ptrs:
            raise ValueError("MasterAdamW.step under HIP graph capture: the parameters moved since "
                             "prepare_graph()")
        table_host, table_dev = self._graph["table_host"], self._graph["table_dev"]
        table_host.copy_(torch.tensor([g.data_ptr() for g in grads], dtype=torch.int64))
        table_dev.copy_(table_host, non_blocking=True)
        _lib.call(
            "nmb_adamw_step_hyper", self._param_table.data_ptr(), table_dev.data_ptr(),
            self.offsets.data_ptr(), len(self.params), self.total, self.master.data_ptr(),
            self.exp_avg.data_ptr(), self.exp_avg_sq.data_ptr(),
            _lib.dtype_code(self.params[0].dtype), _lib.dtype_code(gdtype),
            self._graph["hyper_dev"].data_ptr(), self.max_norm, self.stats.data_ptr(),
            self.workspace.data_ptr(), self.workspace.numel(), _lib.stream_of(self.master),
        )
        self._keep = (grads, table_dev)
