"""The GPT transformer block as two autograd Functions: checkpointed and eager.

Both run the same device sequence (reference GPTLayer.forward,
models/gpt/layer.py:91-137):

    n1 = RMSNorm(x)                          nmb_rmsnorm_fwd
    [q|k|v] = n1 [Wq;Wk;Wv]^T, RoPE(q, k)    nmb_gemm_bf16_rope (RoPE in the epilogue)
    o, lse = attention(q, k, v)              nmb_attn_fwd (MFMA, online softmax)
    h = x + o Wo^T                           nmb_gemm_bf16 with the residual as C input
    n2 = RMSNorm(h)                          nmb_rmsnorm_fwd
    s = silu(n2 Wg^T) * (n2 Wu^T)            nmb_gemm_bf16_swiglu (activation in the epilogue)
    y = h + s Wd^T                           nmb_gemm_bf16 with the residual as C input

``CheckpointedBlockFunction`` is the full-recompute policy of
``activation_checkpoint`` (nn/activation_checkpoint.py:73-100, selected by
models/gpt/model.py:162-170, 215-233): it saves only the block input x.  Its
backward re-runs the sequence above with the same kernels and shapes (so the
recomputed tensors, the attention output and its lse included, are
bit-identical to the forward's) up to n2, and never re-runs the down
projection, whose output the backward does not need.  The gate/up product is
recomputed inside the MLP backward's GEMM (``nmb_gemm_bf16_gate_up_swiglu_bwd``:
per output tile [g|u] = n2 [Wg;Wu]^T, ds = dY Wd and the SwiGLU backward with
all three in registers, the same bits as the forward's gate/up product
followed by the SwiGLU backward; neither [g|u] nor ds reaches memory), which
re-emits s for the Wd gradient.  A block that keeps [g|u] (no checkpoint)
runs the down projection's backward GEMM with the SwiGLU backward as its
epilogue instead (``nmb_gemm_bf16_swiglu_bwd``).  With ``offload`` the saved input goes to
pinned host memory (the reference's saved-tensor offload,
nn/activation_checkpoint.py:24-41); the weights are parameters, never copied.
``EagerBlockFunction`` (activation_checkpoint.mode = "none") keeps the
intermediates instead and shares the backward; ``SelectiveBlockFunction``
("selective") keeps the sub-block inputs and recomputes only the checkpointed
sub-blocks' products.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import Any, Callable

import torch
from torch import Tensor

from nano_megatron_amd import functional as Fn


@dataclass(frozen=True)
class BlockMeta:
    heads: int
    kv_heads: int
    head_dim: int
    eps: float
    sequence_offset: int  # query offset of the causal mask (models/gpt/attention.py:199-206)
    cos: Tensor          # fp32 [n_pos, head_dim/2]
    sin: Tensor
    positions: Tensor | None  # int32 [S] or [B,S], or None for rope_offset + arange
    rope_offset: int | None = None  # RoPE position of token 0 without positions (default: sequence_offset)

    @property
    def pos_offset(self) -> int:
        return self.sequence_offset if self.rope_offset is None else self.rope_offset


def _adjacent(ws: tuple[Tensor, ...]) -> bool:
    """True if the row blocks ws[0], ws[1], ... lie back to back in one storage."""
    w0 = ws[0]
    ptr = w0.data_ptr()
    for w in ws:
        if (not w.is_contiguous() or w.dtype != w0.dtype or w.device != w0.device
                or w.shape[1:] != w0.shape[1:] or w.data_ptr() != ptr
                or w.untyped_storage().data_ptr() != w0.untyped_storage().data_ptr()):
            return False
        ptr += w.numel() * w.element_size()
    return True


def joined(ws: tuple[Tensor, ...]) -> Tensor:
    """The row-concatenation of ws: an alias when they are adjacent, else a copy."""
    if _adjacent(ws):
        rows = sum(w.shape[0] for w in ws)
        return ws[0].as_strided((rows, *ws[0].shape[1:]), ws[0].stride())
    return torch.cat(ws)


def pack_adjacent(params) -> None:
    """Re-home parameters as adjacent row blocks of one buffer (values and
    Parameter objects unchanged), so ``joined`` needs no copy."""
    ws = tuple(p.data for p in params)
    if _adjacent(ws):
        return
    buf = torch.empty(sum(w.shape[0] for w in ws), *ws[0].shape[1:], dtype=ws[0].dtype,
                      device=ws[0].device)
    off = 0
    with torch.no_grad():
        for p in params:
            n = p.shape[0]
            buf[off:off + n].copy_(p.data)
            p.data = buf[off:off + n]
            off += n


def _qkv_views(qkv: Tensor, b: int, s: int, m: BlockMeta) -> tuple[Tensor, Tensor, Tensor]:
    """[B*S, (Hq+2Hkv)*D] -> q [B,S,Hq,D], k, v [B,S,Hkv,D] strided views."""
    qd = m.heads * m.head_dim
    kd = m.kv_heads * m.head_dim
    t = qkv.view(b, s, qkv.shape[-1])
    q = t[:, :, :qd].unflatten(2, (m.heads, m.head_dim))
    k = t[:, :, qd : qd + kd].unflatten(2, (m.kv_heads, m.head_dim))
    v = t[:, :, qd + kd :].unflatten(2, (m.kv_heads, m.head_dim))
    return q, k, v


def _attention_part(n1: Tensor, w: tuple[Tensor, ...], m: BlockMeta, b: int, s: int) -> tuple:
    """[q|k|v] (RoPE applied), the attention output o [B*S, Hq*D] and its lse
    from the normalised block input n1."""
    _, wq, wk, wv = w[:4]
    # Q/K/V projection with RoPE of q and k as the GEMM epilogue
    qkv = Fn.mm_rope(n1, joined((wq, wk, wv)).t(), seq=s, head_dim=m.head_dim,
                     rope_cols=(m.heads + m.kv_heads) * m.head_dim, cos=m.cos, sin=m.sin,
                     pos_offset=m.pos_offset, positions=m.positions)
    q, k, v = _qkv_views(qkv, b, s, m)
    o, lse = Fn.attn_fwd_bshd(q, [k], [v], (0,), causal=True, q_offset=m.sequence_offset, scale=None)
    return qkv, o.view(b * s, m.heads * m.head_dim), lse


def _gate_up_part(n2: Tensor, w: tuple[Tensor, ...], *, act: bool, gu: bool) -> tuple:
    """(s, [g|u]) of the MLP's gate/up product; one GEMM plan whether or not
    the activation is applied in the epilogue, so [g|u] has the same bits."""
    return Fn.mm_gate_up(n2, joined((w[6], w[7])), act=act, gu=gu)


def block_forward(x: Tensor, w: tuple[Tensor, ...], m: BlockMeta, *, recompute: bool,
                  keep_gu: bool = True, gate_up: bool = True) -> dict:
    """Run the block on x [B,S,H].  With recompute=True stop after [g|u] (no s, no y),
    or after n2 with gate_up=False (the backward then recomputes [g|u] inside its
    fused gate/up + SwiGLU-backward GEMM).  With keep_gu=False (a forward whose
    intermediates are dropped) the gate/up GEMM applies the activation in its
    epilogue and [g|u] is never written."""
    w_in, wq, wk, wv, wo, w_post, wg, wu, wd = w
    b, s, hdim = x.shape
    x2 = x.reshape(b * s, hdim)
    n1 = Fn.rmsnorm_fwd(x2, w_in, m.eps)
    qkv, o2, lse = _attention_part(n1, w, m, b, s)
    h = Fn.mm(o2, wo.t(), c=x2, beta=1.0)
    n2 = Fn.rmsnorm_fwd(h, w_post, m.eps)
    acts = dict(x2=x2, n1=n1, qkv=qkv, o2=o2, lse=lse, h=h, n2=n2)
    if recompute and not gate_up:
        return acts
    act, gu = _gate_up_part(n2, w, act=not recompute, gu=recompute or keep_gu)
    if gu is not None:
        acts["gu"] = gu
    if recompute:
        return acts
    acts["s"] = act
    acts["y"] = Fn.mm(act, wd.t(), c=h, beta=1.0).view(b, s, hdim)
    return acts


_SIDE_STREAMS: dict[int, torch.cuda.Stream] = {}


class _SideProducts:
    """Weight-gradient products on a second stream of the device.

    The weight gradients of the block feed nothing else in its backward; on
    their own stream (default priority, like every stream here) they fill the
    CUs that the dX chain's launches leave idle (products of 128-176
    workgroups, split-K tails).  The MLP's two run there; the out-projection's
    and the QKV projection's stay on the main stream: the first's overlap would
    fall on the attention backward, whose workgroups it then displaces, the
    second's on the norm backward only, with the join then holding the next
    layer's recompute (each measured slower on the side).  Each product waits for the work queued so far
    on the main stream, its operands are recorded on the side stream (the
    allocator keeps them until it is done), and ``join`` makes the main stream
    wait for all of them before the gradients are returned (autograd may read
    them on the main stream: accumulation, hooks).  Every kernel is
    deterministic, so the results do not depend on the overlap.  (Letting the
    products run on under the next layers' backward, joined by a final
    callback of the backward pass, measured no faster.)

    Where the products are queued depends on how the step is launched, as
    measured on whole config-3 steps in one process.  Launched from the host,
    the gate/up weight gradient is queued after the dX product that follows
    the fused MLP backward (queued before it, it takes that product's CUs and
    the step is 2.2% slower), and the post-attention norm's dw column sum runs
    on the side.  Captured in a HIP graph, where every cross-stream wait is a
    graph edge that costs device time at each replay (~13 us per layer for the
    wait behind the dX product), the gate/up weight gradient is queued right
    after the down projection's behind the same wait, and the column sum stays
    on the main stream: the replayed step is 1.75% faster."""

    def __init__(self, device: torch.device) -> None:
        self.main = torch.cuda.current_stream(device)
        side = _SIDE_STREAMS.get(device.index)
        if side is None:
            side = _SIDE_STREAMS[device.index] = torch.cuda.Stream(device)
        self.side = side
        self.used = False

    def mm(self, a: Tensor, b: Tensor) -> Tensor:
        self.side.wait_stream(self.main)
        with torch.cuda.stream(self.side):
            out = Fn.mm(a, b)
        a.record_stream(self.side)
        b.record_stream(self.side)
        self.used = True
        return out

    def stream(self) -> torch.cuda.Stream:
        """The side stream for work the caller enqueues there itself (joined
        like the products)."""
        self.used = True
        return self.side

    def join(self) -> None:
        if self.used:
            self.main.wait_stream(self.side)


def block_backward(acts: dict, dy: Tensor, w: tuple[Tensor, ...], m: BlockMeta, shape,
                   prefetch: Callable[[], None] | None = None) -> tuple:
    """Gradients (dx, dw_in, dWq, dWk, dWv, dWo, dw_post, dWg, dWu, dWd) of the
    block.  ``prefetch`` (the recompute prefetch of a captured step) is called
    once the out-projection's products are queued, before the attention
    backward."""
    w_in, wq, wk, wv, wo, w_post, wg, wu, wd = w
    b, s, hdim = shape
    f = wg.shape[0]
    dy2 = dy.reshape(b * s, hdim)
    if not dy2.is_contiguous():
        dy2 = dy2.contiguous()
    x2, n1, qkv, o2, lse, h, n2 = (acts[k] for k in ("x2", "n1", "qkv", "o2", "lse", "h", "n2"))
    side = _SideProducts(dy2.device)

    # MLP: y = h + s Wd^T, s = silu(g) * u, [g|u] = n2 [Wg;Wu]^T
    # ds = dY Wd and the SwiGLU backward in one GEMM (its epilogue); act feeds dWd.
    # Without a kept [g|u] (a recomputed block) the same kernel first forms
    # [g|u] for its tile from n2 (same bits), so the product never reaches memory.
    if "gu" in acts:
        dgu, act = Fn.mm_swiglu_bwd(dy2, wd, acts["gu"])
    else:
        dgu, act = Fn.mm_gate_up_swiglu_bwd(n2, joined((wg, wu)), dy2, wd)
    dwd = side.mm(dy2.t(), act)
    if torch.cuda.is_current_stream_capturing():
        # captured: both MLP weight gradients behind one wait, the column sum
        # on the main stream (fewer cross-stream edges in the graph)
        dwgu = side.mm(dgu.t(), n2)
        dn2 = Fn.mm(dgu, joined((wg, wu)))
        dh, dw_post = Fn.rmsnorm_bwd(h, w_post, dn2, m.eps, residual_grad=dy2)
    else:
        dn2 = Fn.mm(dgu, joined((wg, wu)))
        dwgu = side.mm(dgu.t(), n2)
        # the weight gradient's column sum beside the next products (second stream)
        dh, dw_post = Fn.rmsnorm_bwd(h, w_post, dn2, m.eps, residual_grad=dy2, dw_stream=side.stream())

    # attention: h = x + o Wo^T
    do2 = Fn.mm(dh, wo)
    # on the main stream: beside the attention backward it measured slower
    dwo = Fn.mm(dh.t(), o2)
    if prefetch is not None:
        prefetch()
    q, k, v = _qkv_views(qkv, b, s, m)
    dqkv = torch.empty_like(qkv)
    dq, dk, dv = _qkv_views(dqkv, b, s, m)
    o4 = o2.view(b, s, m.heads, m.head_dim)
    do4 = do2.view(b, s, m.heads, m.head_dim)
    # attention backward with the RoPE backward of q and k fused into the dq/dk stores
    Fn.attn_bwd_rope_bshd(q, k, v, o4, do4, lse, dq, dk, dv, causal=True, q_offset=m.sequence_offset,
                          scale=None, cos=m.cos, sin=m.sin, pos_offset=m.pos_offset,
                          positions=m.positions)
    dn1 = Fn.mm(dqkv, joined((wq, wk, wv)))
    # on the main stream too: on the side it only overlaps the norm backward,
    # and the join then holds the next layer's recompute (measured slower)
    dwqkv = Fn.mm(dqkv.t(), n1)
    dx, dw_in = Fn.rmsnorm_bwd(x2, w_in, dn1, m.eps, residual_grad=dh)
    side.join()

    qd = m.heads * m.head_dim
    kd = m.kv_heads * m.head_dim
    return (
        dx.view(b, s, hdim), dw_in,
        dwqkv[:qd], dwqkv[qd : qd + kd], dwqkv[qd + kd :],
        dwo, dw_post, dwgu[:f], dwgu[f:], dwd,
    )


_PREFETCH_STREAMS: dict[int, torch.cuda.Stream] = {}
# device index -> weak reference to the latest CheckpointedBlockFunction
# context of the forward pass being captured
_LAST_CHECKPOINTED: dict[int, Any] = {}


def begin_forward_pass(device: torch.device) -> None:
    """Called by the model at the start of each forward: the recompute prefetch
    links the checkpointed blocks of one forward pass only."""
    if device.type == "cuda":
        _LAST_CHECKPOINTED.pop(device.index, None)


def _prefetch_recompute(ctx: Any, device: torch.device) -> None:
    """Queues the recompute of the checkpointed block ``ctx`` on a third
    stream; its backward waits for the recorded event, then uses the result.

    In a captured step, a block's backward starts the recompute of the
    checkpointed block before it (in forward order) once its own
    out-projection products are queued, so that the recompute's launches
    overlap the attention backward, the QKV products and the norm backward of
    the block being differentiated instead of following them (replayed config-3
    step -2.1%, same process, bit-identical: the same kernels on the same
    inputs; started before the block's MLP backward instead, -0.7%; launched
    from the host, 2.1% slower, so host-launched steps recompute in place).
    Costs one block's recompute outputs held at the peak."""
    main = torch.cuda.current_stream(device)
    stream = _PREFETCH_STREAMS.get(device.index)
    if stream is None:
        stream = _PREFETCH_STREAMS[device.index] = torch.cuda.Stream(device)
    saved = ctx.saved_tensors
    x, weights = saved[0], tuple(saved[1:])
    stream.wait_stream(main)
    with torch.cuda.stream(stream):
        acts = block_forward(x, weights, ctx.meta, recompute=True, gate_up=False)
        done = torch.cuda.Event()
        done.record(stream)
    ctx.prefetched = (acts, weights, done)


class CheckpointedBlockFunction(torch.autograd.Function):
    """Full per-layer recompute: saves x (the block input) only; with
    ``offload`` x waits for the backward in pinned host memory.  In a captured
    step the recompute of the block before runs early, on a third stream
    (``_prefetch_recompute``)."""

    @staticmethod
    def forward(ctx: Any, x: Tensor, meta: BlockMeta, offload: bool, *weights: Tensor) -> Tensor:
        x = x.contiguous()
        with torch.no_grad():
            acts = block_forward(x, weights, meta, recompute=False, keep_gu=False)
        ctx.meta = meta
        ctx.shape = tuple(x.shape)
        ctx.offloaded = None
        if offload:
            # enqueued after the block's kernels on the same stream, which read x first
            host = torch.empty(x.shape, dtype=x.dtype, pin_memory=True)
            host.copy_(x, non_blocking=True)
            ctx.offloaded = (host, x.device)
            ctx.save_for_backward(*weights)
        else:
            ctx.save_for_backward(x, *weights)
        ctx.prefetched = None
        ctx.prefetch_prev = None
        if not offload and x.is_cuda and torch.cuda.is_current_stream_capturing():
            ctx.prefetch_prev = _LAST_CHECKPOINTED.get(x.device.index)
            _LAST_CHECKPOINTED[x.device.index] = weakref.ref(ctx)
        return acts["y"]

    @staticmethod
    def backward(ctx: Any, dy: Tensor):
        prev = ctx.prefetch_prev() if ctx.prefetch_prev is not None else None
        ctx.prefetch_prev = None
        with torch.no_grad():
            if ctx.prefetched is not None:
                acts, weights, done = ctx.prefetched
                ctx.prefetched = None
                main = torch.cuda.current_stream(dy.device)
                main.wait_event(done)
                for t in acts.values():
                    t.record_stream(main)
            else:
                saved = ctx.saved_tensors
                if ctx.offloaded is not None:
                    host, device = ctx.offloaded
                    x, weights = host.to(device, non_blocking=True), saved
                    ctx.offloaded = None
                else:
                    x, weights = saved[0], saved[1:]
                weights = tuple(weights)
                # the recompute re-runs the forward's attention kernel: o and lse come
                # out bit-identical to the forward's, so the lse needs no saving; the
                # gate/up product is recomputed inside the MLP backward's GEMM
                acts = block_forward(x, weights, ctx.meta, recompute=True, gate_up=False)
            prefetch = None
            if (prev is not None and prev.prefetched is None and prev.offloaded is None
                    and any(prev.needs_input_grad) and torch.cuda.is_current_stream_capturing()):
                prefetch = lambda: _prefetch_recompute(prev, dy.device)  # noqa: E731
            grads = block_backward(acts, dy, weights, ctx.meta, ctx.shape, prefetch=prefetch)
        return (grads[0], None, None, *grads[1:])


class SelectiveBlockFunction(torch.autograd.Function):
    """Selective recompute (activation_checkpoint.mode = "selective",
    models/gpt/layer.py:68-89): the sub-blocks named in ``ops`` ("attention":
    the Q/K/V projection, RoPE, attention and out projection; "mlp": gate/up,
    SwiGLU and down projection) are checkpointed on their inputs, as the
    reference's per-sub-block ``activation_checkpoint`` does.  Saved: the block
    input x and the residual midpoint h (the norms' inputs, outside the
    checkpoints), n1 and n2 (the checkpointed sub-blocks' inputs), and the
    intermediates of a sub-block that is not checkpointed.  The backward
    recomputes a checkpointed attention's [q|k|v], o and lse from n1 and a
    checkpointed MLP's [g|u] from n2 (inside the fused gate/up + SwiGLU
    backward GEMM) with the forward's arithmetic (same bits),
    never the norms, the out projection or the down projection, whose outputs
    it does not read, then runs the shared block backward.  With ``offload``
    the checkpointed sub-blocks' inputs wait in pinned host memory."""

    @staticmethod
    def forward(ctx: Any, x: Tensor, meta: BlockMeta, ops: tuple[str, ...], offload: bool,
                *weights: Tensor) -> Tensor:
        x = x.contiguous()
        attn_ck, mlp_ck = "attention" in ops, "mlp" in ops
        with torch.no_grad():
            acts = block_forward(x, weights, meta, recompute=False, keep_gu=not mlp_ck)
        ctx.meta = meta
        ctx.shape = tuple(x.shape)
        ctx.ops = (attn_ck, mlp_ck)
        keep = ["h"] + ([] if attn_ck else ["n1", "qkv", "o2", "lse"]) + ([] if mlp_ck else ["n2", "gu"])
        ck = ([acts["n1"]] if attn_ck else []) + ([acts["n2"]] if mlp_ck else [])
        ctx.keys = keep
        ctx.offloaded = None
        if offload and ck:
            # enqueued after the block's kernels on the same stream, which read them first
            host = [torch.empty(t.shape, dtype=t.dtype, pin_memory=True) for t in ck]
            for hst, t in zip(host, ck):
                hst.copy_(t, non_blocking=True)
            ctx.offloaded = (host, x.device)
            ck = []
        ctx.n_ck = len(ck)
        ctx.save_for_backward(x, *(acts[k] for k in keep), *ck, *weights)
        return acts["y"]

    @staticmethod
    def backward(ctx: Any, dy: Tensor):
        saved = ctx.saved_tensors
        x, weights = saved[0], tuple(saved[1 + len(ctx.keys) + ctx.n_ck:])
        acts = dict(zip(ctx.keys, saved[1:1 + len(ctx.keys)]))
        ck = list(saved[1 + len(ctx.keys):1 + len(ctx.keys) + ctx.n_ck])
        if ctx.offloaded is not None:
            host, device = ctx.offloaded
            ck = [t.to(device, non_blocking=True) for t in host]
            ctx.offloaded = None
        attn_ck, mlp_ck = ctx.ops
        b, s, hdim = ctx.shape
        m = ctx.meta
        acts["x2"] = x.reshape(b * s, hdim)
        with torch.no_grad():
            if attn_ck:
                acts["n1"] = ck.pop(0)
                acts["qkv"], acts["o2"], acts["lse"] = _attention_part(acts["n1"], weights, m, b, s)
            if mlp_ck:
                # [g|u] is recomputed inside the MLP backward's GEMM
                acts["n2"] = ck.pop(0)
            grads = block_backward(acts, dy, weights, m, ctx.shape)
        return (grads[0], None, None, None, *grads[1:])


class EagerBlockFunction(torch.autograd.Function):
    """No checkpoint: keeps every intermediate the backward reads."""

    @staticmethod
    def forward(ctx: Any, x: Tensor, meta: BlockMeta, *weights: Tensor) -> Tensor:
        with torch.no_grad():
            acts = block_forward(x.contiguous(), weights, meta, recompute=False)
        ctx.meta = meta
        ctx.shape = tuple(x.shape)
        keys = ("x2", "n1", "qkv", "o2", "lse", "h", "n2", "gu")
        ctx.keys = keys
        ctx.save_for_backward(*(acts[k] for k in keys), *weights)
        return acts["y"]

    @staticmethod
    def backward(ctx: Any, dy: Tensor):
        saved = ctx.saved_tensors
        n = len(ctx.keys)
        acts = dict(zip(ctx.keys, saved[:n]))
        weights = tuple(saved[n:])
        with torch.no_grad():
            grads = block_backward(acts, dy, weights, ctx.meta, ctx.shape)
        return (grads[0], None, *grads[1:])
