"""A training step captured once as a HIP graph and replayed.

The trainer's step (reference training/trainer.py:424-474: zero_grad, the
forward with labels, backward, the optimizer step) launches every kernel from
the host, ~870 of them per step at config 3.  ``CapturedTrainStep`` records the
same step once with ``torch.cuda.graph`` and replays it: the same kernels on
the same buffers, in the same order, so a replay computes bit-identically to an
eager step (tested), with one launch from the host and without the gaps the
device leaves between separately launched kernels.

What changes per replay and what does not:
- the batch: ``step(input_ids, labels)`` copies it into the graph's input
  buffers (fixed shapes);
- the optimizer's step count, hence its bias corrections and learning rate:
  ``MasterAdamW.advance_graph_step`` writes them to a device record that the
  captured update reads;
- the target check (ids outside [0, vocab) raise ``ValueError`` before the
  update, as in the eager forward, tensor_parallel/cross_entropy.py:109-114):
  made before each replay, since a host wait cannot be captured.
The activation checkpoint options must not move tensors to the host
(``offload_saved_tensors``) nor recompute under ``torch.utils.checkpoint``
(a layer outside the fused block in mode "full" or "selective"), explicit ``position_ids`` (read on the host) are
not accepted, and neither is dropout > 0 (its masks are keyed by seeds passed
at launch, which every replay would repeat); all raise ``ValueError``.  No reference to an earlier step's
autograd graph (an undetached loss) may be alive when the step is captured:
its gradient-accumulation nodes belong to the stream of that earlier step,
and the backward under capture would synchronise with it, which invalidates
the capture.
"""

from __future__ import annotations

import torch
from torch import Tensor

from nano_megatron_amd import functional as Fn
from nano_megatron_amd.optim import MasterAdamW


class CapturedTrainStep:
    def __init__(self, model: torch.nn.Module, optimizer: MasterAdamW, input_ids: Tensor,
                 labels: Tensor) -> None:
        if not (input_ids.is_cuda and labels.is_cuda):
            raise ValueError("CapturedTrainStep runs on the GPU: input_ids and labels must be HIP tensors")
        if not isinstance(optimizer, MasterAdamW):
            raise ValueError("CapturedTrainStep needs a MasterAdamW optimizer (its update reads "
                             "per-step scalars from device memory)")
        ckpt = getattr(model, "activation_checkpoint_config", None)
        if bool(getattr(ckpt, "offload_saved_tensors", False)):
            raise ValueError("offload_saved_tensors copies to host memory, which a HIP graph "
                             "replay cannot reuse: capture without it")
        if getattr(model, "lm_head", None) is None:
            raise ValueError("CapturedTrainStep needs the stage that owns the LM head (the loss)")
        rates = (getattr(m, "dropout", 0.0) for m in model.modules())
        if any(isinstance(r, (int, float)) and not isinstance(r, bool) and r > 0.0 for r in rates):
            raise ValueError("dropout masks are keyed by seeds passed from the host at launch, which "
                             "every replay of a captured graph would repeat: capture with dropout 0")
        mode = getattr(ckpt, "mode", "none")
        if mode in ("full", "selective") and any(not layer.fusable() for layer in getattr(model, "layers", ())):
            raise ValueError("a layer outside the fused block (biases, other head sizes or components) "
                             "recomputes under torch.utils.checkpoint, whose RNG-state replay cannot be "
                             f"captured: capture with activation_checkpoint.mode 'none' or fused layers only "
                             f"(mode {mode!r})")
        self.model, self.optimizer = model, optimizer
        self.device = input_ids.device
        self.vocab = model.lm_head.weight.shape[0]
        self.input_ids = input_ids.detach().clone()
        self.labels = labels.detach().clone()
        self.loss = torch.zeros((), dtype=torch.float32, device=self.device)
        Fn.TargetCheck(self.labels, self.vocab, Fn.IGNORE_INDEX).raise_if_invalid()
        self._labels_checked = True  # the labels buffer holds checked targets

        # One forward and backward outside the capture, on a side stream, for the
        # device state the first call creates (packed block weights, RoPE
        # tables, the weight-gradient stream); the gradients are dropped and
        # the weights are unchanged.
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            optimizer.zero_grad()
            model(self.input_ids, labels=self.labels).loss.backward()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        optimizer.zero_grad()
        optimizer.prepare_graph()

        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            optimizer.zero_grad()
            loss = model(self.input_ids, labels=self.labels).loss
            loss.backward()
            optimizer.step()
            self.loss.copy_(loss.detach())

    def step(self, input_ids: Tensor | None = None, labels: Tensor | None = None) -> Tensor:
        """One training step on the batch (the previous one when omitted).  New
        labels are copied in and checked before the replay (the host waits for
        the check, hence for the previous replay, and raises the ValueError
        before any update); labels already checked are not checked again, and
        the replay is then queued behind the previous one without a host wait.
        Returns the loss (a device scalar, overwritten by the next replay)."""
        if input_ids is not None:
            if input_ids.shape != self.input_ids.shape:
                raise ValueError(f"input_ids shape {tuple(input_ids.shape)} differs from the captured "
                                 f"{tuple(self.input_ids.shape)}")
            self.input_ids.copy_(input_ids)
        if labels is not None:
            if labels.shape != self.labels.shape:
                raise ValueError(f"labels shape {tuple(labels.shape)} differs from the captured "
                                 f"{tuple(self.labels.shape)}")
            self._labels_checked = False
            self.labels.copy_(labels)
        if not self._labels_checked:
            Fn.TargetCheck(self.labels, self.vocab, Fn.IGNORE_INDEX).raise_if_invalid()
            self._labels_checked = True
        self.optimizer.advance_graph_step()
        self.graph.replay()
        return self.loss
