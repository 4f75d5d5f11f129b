"""Device ops of the GPT block: thin wrappers over libnmb.so plus autograd Functions.

Every op runs on the GPU through the C ABI; a CPU tensor is an error, never a
fallback.  Every bf16 op, the dense projections included, is a hand-written
gfx950 kernel; fp32 (the parity configuration) projections use the library
GEMM.

Attention tensors use one memory layout throughout: ``[batch, seq, heads,
head_dim]`` (the layout of the Q/K/V projection outputs), seen through a
``[batch, heads, seq, head_dim]`` view where the reference API expects it
(nn/kernels/torch_backend.py:25-76).  That makes the reference's
``transpose(1, 2).contiguous()`` (models/gpt/attention.py:176-178, 207) free.
"""

from __future__ import annotations

import math
import threading
from typing import Any, Sequence

import torch
from torch import Tensor

from nano_megatron_amd import _lib

IGNORE_INDEX = -100


def _require_gpu(*tensors: Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(
                "nano_megatron_amd runs its kernels on the GPU only; got a tensor on "
                f"{t.device} (there is no CPU fallback)"
            )


SUPPORTED_PRECISIONS = (
    "params=float32 with compute=float32, or params=bfloat16 with compute=bfloat16 "
    "(bf16 parameters and activations, the fp32-master optimizer; torch.autocast to bfloat16 "
    "around it is accepted)"
)


def require_precision(*tensors: Tensor) -> None:
    """The precision modes these kernels implement (config/schema.py:55-64,
    training/trainer.py:49-57): every kernel computes in its inputs' dtype,
    float32 or bfloat16.  Two reference modes are refused with a ValueError
    instead of running something else silently: float16 (no kernels), and
    float32 parameters under ``torch.autocast`` to a lower dtype (the
    reference's params=float32/compute=bfloat16 mode, where autocast runs the
    linears and attention in bf16 on an fp32 residual stream; these kernels
    would run them in fp32)."""
    for t in tensors:
        if t is None:
            continue
        if t.dtype == torch.float16:
            raise ValueError(f"precision float16 has no kernels in nano_megatron_amd; supported: "
                             f"{SUPPORTED_PRECISIONS}")
        device_type = t.device.type
        if torch.is_autocast_enabled(device_type):
            cast = torch.get_autocast_dtype(device_type)
            if t.is_floating_point() and cast != t.dtype:
                raise ValueError(
                    f"torch.autocast({device_type}, dtype={cast}) around {t.dtype} tensors is the "
                    f"reference's params={str(t.dtype).replace('torch.', '')}/compute="
                    f"{str(cast).replace('torch.', '')} mode, which these kernels do not implement "
                    f"(they compute in the tensors' own dtype); supported: {SUPPORTED_PRECISIONS}")


def _workspace(nbytes: int, device: torch.device) -> Tensor:
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------- GEMM
_GEMM_WS: dict = {}  # (layouts, m, n, k) -> split-K workspace bytes (a pure function of the shape)


def _operand_layout(t: Tensor, rows_dim: int) -> tuple[int, int]:
    """(layout, ld) of a 2-D operand: 0 if dim 1 is contiguous (ld = stride(0)),
    1 if dim 0 is contiguous (ld = stride(1))."""
    if t.stride(1) == 1 and (t.shape[0] == 1 or t.stride(0) >= t.shape[1]):
        return 0, max(t.stride(0), t.shape[1])
    if t.stride(0) == 1 and (t.shape[1] == 1 or t.stride(1) >= t.shape[0]):
        return 1, max(t.stride(1), t.shape[0])
    raise ValueError("gemm operands need one contiguous dimension")


def mm(a: Tensor, b: Tensor, *, out: Tensor | None = None, c: Tensor | None = None,
       alpha: float = 1.0, beta: float = 0.0) -> Tensor:
    """``out = alpha * a @ b + beta * c`` for 2-D tensors (``c`` may be ``out``).

    bf16 runs the gfx950 MFMA kernel ``nmb_gemm_bf16``, fp32 (the parity
    configuration) the fp32-MFMA kernel ``nmb_gemm_f32``; both take any mix of
    row/column-major operands.  Other dtypes are a ValueError.
    """
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError(f"gemm: inner dimensions differ ({k} vs {k2})")
    if a.dtype != b.dtype or (c is not None and c.dtype != a.dtype):
        raise ValueError(f"gemm: operands of one dtype needed, got {a.dtype}, {b.dtype}")
    if out is None:
        out = torch.empty(m, n, dtype=a.dtype, device=a.device)
    if a.dtype == torch.float32:
        return _mm_f32(a, b, out, c, alpha, beta)
    if a.dtype != torch.bfloat16:
        raise ValueError(f"nano_megatron_amd GEMMs support float32 and bfloat16, got {a.dtype}")
    _require_gpu(a, b, out)
    la, lda = _operand_layout(a, 0)
    # B is [K, N]: layout 0 means stored [N, K] (dim 0 = K contiguous)
    lb_rowmajor, ldb = _operand_layout(b, 0)
    lb = 1 - lb_rowmajor
    if out.stride(1) != 1:
        raise ValueError("gemm: the output must be row-major")
    if beta != 0.0 and (c is None or c.stride(1) != 1):
        raise ValueError("gemm: beta != 0 needs a row-major C")
    key = (la, lb, m, n, k)
    nbytes = _GEMM_WS.get(key)
    if nbytes is None:
        q = _lib.ctypes.c_int64()
        _lib.call("nmb_gemm_bf16_workspace_bytes", la, lb, m, n, k, _lib.ctypes.byref(q))
        nbytes = _GEMM_WS[key] = q.value
    ws = _workspace(nbytes, a.device) if nbytes else None
    _lib.call(
        "nmb_gemm_bf16", la, lb, m, n, k, float(alpha), a.data_ptr(), lda, b.data_ptr(), ldb,
        float(beta), _lib.ptr(c), c.stride(0) if c is not None else n, out.data_ptr(),
        out.stride(0), _lib.ptr(ws), ws.numel() if ws is not None else 0, _lib.stream_of(a),
    )
    return out


def mm_f32out(a: Tensor, b: Tensor, out: Tensor, *, alpha: float = 1.0, beta: float = 0.0) -> Tensor:
    """``out = alpha * a @ b + beta * out`` with bf16 ``a``, ``b`` and an fp32
    row-major ``out`` (``nmb_gemm_bf16_f32out``): sums of bf16 products kept
    in fp32, to be rounded once by the caller."""
    m, k = a.shape
    k2, n = b.shape
    if k != k2 or out.shape != (m, n):
        raise ValueError(f"gemm_f32out: shapes {tuple(a.shape)} x {tuple(b.shape)} -> {tuple(out.shape)}")
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16 or out.dtype != torch.float32:
        raise ValueError("gemm_f32out: bf16 operands and an fp32 output needed")
    _require_gpu(a, b, out)
    if out.stride(1) != 1:
        raise ValueError("gemm_f32out: the output must be row-major")
    la, lda = _operand_layout(a, 0)
    lb_rowmajor, ldb = _operand_layout(b, 0)
    lb = 1 - lb_rowmajor
    key = (la, lb, m, n, k)
    nbytes = _GEMM_WS.get(key)
    if nbytes is None:
        q = _lib.ctypes.c_int64()
        _lib.call("nmb_gemm_bf16_workspace_bytes", la, lb, m, n, k, _lib.ctypes.byref(q))
        nbytes = _GEMM_WS[key] = q.value
    ws = _workspace(nbytes, a.device) if nbytes else None
    _lib.call(
        "nmb_gemm_bf16_f32out", la, lb, m, n, k, float(alpha), a.data_ptr(), lda, b.data_ptr(), ldb,
        float(beta), out.data_ptr(), out.stride(0), _lib.ptr(ws), ws.numel() if ws is not None else 0,
        _lib.stream_of(a),
    )
    return out


def _any_layout(t: Tensor) -> tuple[Tensor, int, int]:
    """(t or a contiguous copy, layout, ld) for an fp32 operand (layout as _operand_layout)."""
    try:
        la, ld = _operand_layout(t, 0)
    except ValueError:
        t = t.contiguous()
        la, ld = _operand_layout(t, 0)
    return t, la, ld


def _mm_f32(a: Tensor, b: Tensor, out: Tensor, c: Tensor | None, alpha: float, beta: float) -> Tensor:
    _require_gpu(a, b, out)
    m, k = a.shape
    n = b.shape[1]
    a, la, lda = _any_layout(a)
    b, lb_rowmajor, ldb = _any_layout(b)
    if out.stride(1) != 1 and out.numel() > 1:
        raise ValueError("gemm: the output must be row-major")
    if beta != 0.0 and (c is None or (c.stride(1) != 1 and c.numel() > 1)):
        raise ValueError("gemm: beta != 0 needs a row-major C")
    _lib.call(
        "nmb_gemm_f32", la, 1 - lb_rowmajor, m, n, k, float(alpha), a.data_ptr(), lda, b.data_ptr(),
        ldb, float(beta), _lib.ptr(c) if beta != 0.0 else None,
        max(c.stride(0), n) if (c is not None and beta != 0.0) else n, out.data_ptr(),
        max(out.stride(0), n), _lib.stream_of(a),
    )
    return out


def _round8(n: int) -> int:
    return (n + 7) // 8 * 8


def _zero_padded(t: Tensor, rows: int, cols: int) -> Tensor:
    """``t`` (2-D) in the top-left corner of a zero [rows, cols] tensor."""
    if tuple(t.shape) == (rows, cols):
        return t
    out = torch.zeros(rows, cols, dtype=t.dtype, device=t.device)
    out[: t.shape[0], : t.shape[1]].copy_(t)
    return out


class LinearFunction(torch.autograd.Function):
    """``F.linear(x, weight)`` (nn/kernels/torch_backend.py:19-20,
    tensor_parallel/layers.py:214) on the library's GEMMs: y = x W^T,
    dX = dY W, dW = dY^T X.  The bf16 GEMM moves 16-byte chunks, so feature
    counts that are not multiples of 8 (a 50257-token vocabulary, say) run on
    copies zero-padded to the next multiple of 8: the extra terms are zero
    products, so the results are those of the unpadded shapes."""

    @staticmethod
    def forward(ctx: Any, x: Tensor, weight: Tensor) -> Tensor:
        if x.shape[-1] != weight.shape[1]:
            raise ValueError(f"linear: input features {x.shape[-1]} != weight {weight.shape[1]}")
        x2 = x.reshape(-1, x.shape[-1])
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        n, k = weight.shape
        ctx.save_for_backward(x2, weight)
        ctx.shape = x.shape
        if weight.dtype == torch.bfloat16 and (n % 8 or k % 8):
            n8, k8 = _round8(n), _round8(k)
            y = mm(_zero_padded(x2, x2.shape[0], k8), _zero_padded(weight, n8, k8).t())[:, :n].contiguous()
        else:
            y = mm(x2, weight.t())
        return y.view(*x.shape[:-1], n)

    @staticmethod
    def backward(ctx: Any, dy: Tensor):
        x2, weight = ctx.saved_tensors
        n, k = weight.shape
        dy2 = dy.reshape(-1, n)
        if not dy2.is_contiguous():
            dy2 = dy2.contiguous()
        dx = dw = None
        if weight.dtype == torch.bfloat16 and (n % 8 or k % 8):
            n8, k8 = _round8(n), _round8(k)
            dyp = _zero_padded(dy2, dy2.shape[0], n8)
            if ctx.needs_input_grad[0]:
                dx = mm(dyp, _zero_padded(weight, n8, k8))[:, :k].contiguous().view(ctx.shape)
            if ctx.needs_input_grad[1]:
                dw = mm(dyp.t(), _zero_padded(x2, x2.shape[0], k8))[:n, :k].contiguous()
            return dx, dw
        if ctx.needs_input_grad[0]:
            dx = mm(dy2, weight).view(ctx.shape)
        if ctx.needs_input_grad[1]:
            dw = mm(dy2.t(), x2)
        return dx, dw


def linear(x: Tensor, weight: Tensor, bias: Tensor | None = None) -> Tensor:
    """``F.linear`` with the GEMM on this library's kernels (the bias, when a
    module has one, is added by a broadcast tensor add)."""
    require_precision(x, weight)
    y = LinearFunction.apply(x, weight)
    return y if bias is None else y + bias


def mm_rope(a: Tensor, b: Tensor, *, seq: int, head_dim: int, rope_cols: int, cos: Tensor,
            sin: Tensor, pos_offset: int = 0, positions: Tensor | None = None,
            out: Tensor | None = None) -> Tensor:
    """``a @ b`` with RoPE applied to the first ``rope_cols`` output columns
    (heads of ``head_dim``; row r is token (r // seq, r % seq)), as the Q/K/V
    projection followed by the rotary embedding of q and k
    (models/gpt/attention.py:172-181).  bf16 runs the fused GEMM epilogue
    ``nmb_gemm_bf16_rope`` (heads of 64 or 128); otherwise the GEMM and then the
    rotary kernel."""
    m, k = a.shape
    n = b.shape[1]
    if rope_cols % head_dim or rope_cols > n or m % seq:
        raise ValueError("mm_rope: rope_cols must be whole heads within N and M = batch x seq")
    if a.dtype != torch.bfloat16 or head_dim not in (64, 128):
        # the fused epilogue covers bf16 heads of 64 and 128; otherwise GEMM, then rotary kernel
        out = mm(a, b, out=out)
        x = out.view(m // seq, seq, n)[:, :, :rope_cols].unflatten(2, (rope_cols // head_dim, head_dim))
        rope_apply(x, x, cos, sin, pos_offset=pos_offset, positions=positions)
        return out
    _require_gpu(a, b, cos, sin)
    if out is None:
        out = torch.empty(m, n, dtype=a.dtype, device=a.device)
    elif out.shape != (m, n) or out.dtype != a.dtype or out.stride(1) != 1:
        raise ValueError("mm_rope: out must be a row-major [M, N] tensor of a's dtype")
    la, lda = _operand_layout(a, 0)
    if la != 0:
        raise ValueError("mm_rope: a must be row-major")
    lb_rowmajor, ldb = _operand_layout(b, 0)
    pos_ptr, pos_bstride = None, 0
    if positions is not None:
        if positions.dtype != torch.int32:
            raise ValueError("mm_rope: positions must be int32")
        pos_ptr = positions.data_ptr()
        pos_bstride = positions.stride(0) if positions.ndim == 2 else 0
    _lib.call(
        "nmb_gemm_bf16_rope", 1 - lb_rowmajor, m, n, k, a.data_ptr(), lda, b.data_ptr(), ldb,
        out.data_ptr(), out.stride(0), cos.data_ptr(), sin.data_ptr(), cos.shape[0], pos_ptr,
        pos_bstride, int(pos_offset), seq, head_dim, rope_cols, _lib.stream_of(a),
    )
    return out


# ---------------------------------------------------------------- RMSNorm
def rmsnorm_fwd(x2: Tensor, weight: Tensor, eps: float) -> Tensor:
    """y = RMSNorm(x2) for a contiguous [rows, hidden] tensor (nn/norms.py:38-41)."""
    _require_gpu(x2, weight)
    rows, cols = x2.shape
    y = torch.empty_like(x2)
    _lib.call(
        "nmb_rmsnorm_fwd", x2.data_ptr(), weight.data_ptr(), y.data_ptr(), None, rows, cols,
        float(eps), _lib.dtype_code(x2.dtype), _lib.stream_of(x2),
    )
    return y


def rmsnorm_bwd(
    x2: Tensor, weight: Tensor, dy2: Tensor, eps: float, residual_grad: Tensor | None = None,
    dw_stream: "torch.cuda.Stream | None" = None,
) -> tuple[Tensor, Tensor]:
    """(dx [+ residual_grad], dw) of RMSNorm, with dw reduced deterministically.
    With ``dw_stream`` the weight gradient's column sum runs there, after the
    current stream's work so far (the caller joins that stream before dw is
    read on another); the bits are the same."""
    _require_gpu(x2, weight, dy2)
    rows, cols = x2.shape
    nbytes = _lib.ctypes.c_size_t(0)
    _lib.call("nmb_rmsnorm_bwd_workspace_bytes", rows, cols, _lib.ctypes.byref(nbytes))
    ws = _workspace(nbytes.value, x2.device)
    dx = torch.empty_like(x2)
    dw = torch.empty_like(weight)
    code = _lib.dtype_code(x2.dtype)
    if dw_stream is None:
        _lib.call(
            "nmb_rmsnorm_bwd", x2.data_ptr(), weight.data_ptr(), dy2.data_ptr(),
            _lib.ptr(residual_grad), dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), ws.numel(),
            rows, cols, float(eps), code, _lib.stream_of(x2),
        )
        return dx, dw
    _lib.call(
        "nmb_rmsnorm_bwd_rows", x2.data_ptr(), weight.data_ptr(), dy2.data_ptr(),
        _lib.ptr(residual_grad), dx.data_ptr(), ws.data_ptr(), ws.numel(), rows, cols, float(eps), code,
        _lib.stream_of(x2),
    )
    dw_stream.wait_stream(torch.cuda.current_stream(x2.device))
    _lib.call("nmb_rmsnorm_bwd_dw", ws.data_ptr(), ws.numel(), rows, cols, dw.data_ptr(), code,
              dw_stream.cuda_stream)
    ws.record_stream(dw_stream)
    dw.record_stream(dw_stream)
    return dx, dw


class RMSNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, x: Tensor, weight: Tensor, eps: float) -> Tensor:
        if x.shape[-1] != weight.shape[0]:
            raise ValueError(f"expected the last dimension to be {weight.shape[0]}, got {x.shape[-1]}")
        if weight.dtype != x.dtype:
            weight = weight.to(x.dtype)
        x2 = x.reshape(-1, x.shape[-1]).contiguous()
        y = rmsnorm_fwd(x2, weight.contiguous(), eps)
        ctx.save_for_backward(x2, weight)
        ctx.eps = eps
        ctx.shape = x.shape
        return y.view(x.shape)

    @staticmethod
    def backward(ctx: Any, dy: Tensor):
        x2, weight = ctx.saved_tensors
        dx, dw = rmsnorm_bwd(x2, weight, dy.reshape(x2.shape).contiguous(), ctx.eps)
        return dx.view(ctx.shape), dw, None


def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    require_precision(x, weight)
    return RMSNormFunction.apply(x, weight, eps)


# ---------------------------------------------------------------- RoPE tables
class RopeTables:
    """fp32 cos/sin tables [n_pos, head_dim/2] on one device, grown on demand.

    ``inv_freq`` is computed on the host exactly as nn/rotary.py:52 does; the
    table rows are ``cos(p * inv_freq)`` / ``sin(p * inv_freq)`` computed by
    ``nmb_rope_table``.  Because ``emb = cat(f, f)`` only half a row is kept.
    """

    _cache: dict[tuple, "RopeTables"] = {}
    _lock = threading.Lock()

    def __init__(self, device: torch.device, head_dim: int, theta: float) -> None:
        self.device = device
        self.head_dim = head_dim
        self.theta = theta
        inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        self.inv_freq = inv.to(device)
        self.n_pos = 0
        self.cos = self.sin = None

    @classmethod
    def get(cls, device: torch.device, head_dim: int, theta: float, n_pos: int) -> "RopeTables":
        key = (device.type, device.index, head_dim, float(theta))
        with cls._lock:
            tab = cls._cache.get(key)
            if tab is None:
                tab = cls._cache[key] = RopeTables(device, head_dim, theta)
            tab._ensure(n_pos)
            return tab

    def _ensure(self, n_pos: int) -> None:
        if n_pos <= self.n_pos:
            return
        if self.device.type != "cuda":
            raise ValueError("RoPE tables are built on the GPU only (there is no CPU fallback)")
        n = 1 << max(10, int(math.ceil(math.log2(max(n_pos, 1)))))
        half = self.head_dim // 2
        cos = torch.empty(n, half, dtype=torch.float32, device=self.device)
        sin = torch.empty_like(cos)
        _lib.call(
            "nmb_rope_table", cos.data_ptr(), sin.data_ptr(), self.inv_freq.data_ptr(), n, half,
            _lib.stream_of(cos),
        )
        self.cos, self.sin, self.n_pos = cos, sin, n


def rope_apply(
    x: Tensor,
    out: Tensor,
    cos: Tensor,
    sin: Tensor,
    *,
    pos_offset: int = 0,
    positions: Tensor | None = None,
    inverse: bool = False,
) -> None:
    """Rotate x [B, S, H, D] (any strides, last dim contiguous) into out.

    cos/sin are fp32 [n_pos, D/2] tables; position of (b, s) is
    positions[b, s] (int32 [S] or [B, S]) or pos_offset + s.
    """
    _require_gpu(x, out, cos, sin)
    b, s, h, d = x.shape
    if x.stride(3) != 1 or out.stride(3) != 1:
        raise ValueError("rope_apply: head_dim must be the contiguous dimension")
    pos_ptr, pos_bstride = None, 0
    if positions is not None:
        if positions.dtype != torch.int32:
            raise ValueError("rope_apply: positions must be int32")
        pos_ptr = positions.data_ptr()
        pos_bstride = positions.stride(0) if positions.ndim == 2 else 0
    _lib.call(
        "nmb_rope_apply", x.data_ptr(), out.data_ptr(), cos.data_ptr(), sin.data_ptr(),
        cos.shape[0], pos_ptr, pos_bstride, int(pos_offset), b, s, h, d,
        _lib.i64x3((x.stride(0), x.stride(1), x.stride(2))),
        _lib.i64x3((out.stride(0), out.stride(1), out.stride(2))),
        1 if inverse else 0, _lib.dtype_code(x.dtype), _lib.stream_of(x),
    )


def _bshd_view(t_bhsd: Tensor) -> Tensor:
    """[B,H,S,D] tensor -> [B,S,H,D] view of the same memory."""
    return t_bhsd.transpose(1, 2)


def _new_bhsd(shape_bhsd: Sequence[int], like: Tensor) -> Tensor:
    """Allocate a [B,H,S,D] tensor stored as [B,S,H,D] memory."""
    b, h, s, d = shape_bhsd
    return torch.empty(b, s, h, d, dtype=like.dtype, device=like.device).transpose(1, 2)


def _eff_strides(t: Tensor, dims=(0, 1, 2)) -> tuple[int, ...]:
    """Strides of the given dims with size-1 dims reported as 0 (never multiplied
    by a non-zero index, so any stride is equivalent there)."""
    return tuple(t.stride(i) if t.shape[i] > 1 else 0 for i in dims)


def _canonical_bhsd(t: Tensor) -> Tensor:
    """Return t ([B,H,S,D]) with [B,S,H,D]-contiguous memory, copying only if needed."""
    b, h, s, d = t.shape
    want = tuple(st if n > 1 else 0 for st, n in zip((s * h * d, d, h * d, 1), (b, h, s, d)))
    if t.numel() == 0 or _eff_strides(t, (0, 1, 2, 3)) == want:
        return t
    return t.transpose(1, 2).contiguous().transpose(1, 2)


class RotaryFunction(torch.autograd.Function):
    """``q*cos + rotate_half(q)*sin`` for one [B,H,S,D] tensor, backward by -theta."""

    @staticmethod
    def forward(ctx: Any, x: Tensor, cos: Tensor, sin: Tensor, positions: Tensor | None,
                pos_offset: int) -> Tensor:
        out = _new_bhsd(x.shape, x)
        rope_apply(_bshd_view(x), _bshd_view(out), cos, sin, pos_offset=pos_offset,
                   positions=positions)
        ctx.save_for_backward(cos, sin, positions)
        ctx.pos_offset = pos_offset
        return out

    @staticmethod
    def backward(ctx: Any, grad: Tensor):
        cos, sin, positions = ctx.saved_tensors
        grad = _canonical_bhsd(grad)
        dx = _new_bhsd(grad.shape, grad)
        rope_apply(_bshd_view(grad), _bshd_view(dx), cos, sin, pos_offset=ctx.pos_offset,
                   positions=positions, inverse=True)
        return dx, None, None, None, None


def rope_tables_from_cos_sin(
    cos: Tensor, sin: Tensor, batch: int, seq: int
) -> tuple[Tensor, Tensor, Tensor]:
    """Turn reference-style cos/sin ([S,D] or [B,S,D], emb = cat(f, f)) into
    fp32 half tables plus an int32 row index per (b, s)."""
    half = cos.shape[-1] // 2
    if cos.ndim == 2:
        ct = cos[:, :half].float().contiguous()
        st = sin[:, :half].float().contiguous()
        pos = torch.arange(seq, dtype=torch.int32, device=cos.device)
    elif cos.ndim == 3:
        ct = cos[..., :half].float().reshape(-1, half).contiguous()
        st = sin[..., :half].float().reshape(-1, half).contiguous()
        pos = torch.arange(cos.shape[0] * seq, dtype=torch.int32, device=cos.device).view(-1, seq)
    else:
        raise ValueError(
            "RoPE cos/sin tensors must have shape [sequence, head_dim] or "
            f"[batch, sequence, head_dim], got {tuple(cos.shape)}"
        )
    return ct, st, pos


# ---------------------------------------------------------------- SwiGLU
def swiglu_fwd(g: Tensor, u: Tensor, out: Tensor | None = None) -> Tensor:
    _require_gpu(g, u)
    rows, cols = g.shape
    if out is None:
        out = torch.empty(rows, cols, dtype=g.dtype, device=g.device)
    _lib.call(
        "nmb_swiglu_fwd", g.data_ptr(), g.stride(0), u.data_ptr(), u.stride(0), out.data_ptr(),
        out.stride(0), rows, cols, _lib.dtype_code(g.dtype), _lib.stream_of(g),
    )
    return out


def mm_swiglu_bwd(dy: Tensor, wd: Tensor, gu: Tensor, *, act: bool = True) -> tuple[Tensor, Tensor | None]:
    """The MLP's backward through the down projection and SwiGLU (autograd of
    models/gpt/mlp.py:77-78): ``ds = dy @ wd`` (``wd`` the down projection's
    [H, F] weight), then the SwiGLU backward against the forward's gate/up
    product ``gu`` [M, 2F].  Returns (``dgu`` [M, 2F] = (d gate | d up), the
    activation ``silu(g) * u`` [M, F] if act).  bf16 runs one GEMM with the
    SwiGLU backward as its epilogue (``nmb_gemm_bf16_swiglu_bwd``, bit-identical
    to the product then ``swiglu_bwd``, without ds in memory); other dtypes run
    the two."""
    m, h = dy.shape
    h2, f = wd.shape
    if h != h2 or gu.shape != (m, 2 * f):
        raise ValueError("mm_swiglu_bwd: dy [M, H], wd [H, F] and gu [M, 2F] expected")
    dgu = torch.empty_like(gu)
    out = torch.empty(m, f, dtype=gu.dtype, device=gu.device) if act else None
    if dy.dtype != torch.bfloat16:
        ds = mm(dy, wd)
        o = out if out is not None else torch.empty(m, f, dtype=gu.dtype, device=gu.device)
        swiglu_bwd(gu[:, :f], gu[:, f:], ds, dgu[:, :f], dgu[:, f:], o)
        return dgu, out
    _require_gpu(dy, wd, gu)
    if dy.stride(1) != 1 or wd.stride(1) != 1 or gu.stride(1) != 1 or not (dy.dtype == wd.dtype == gu.dtype):
        raise ValueError("mm_swiglu_bwd: dy, wd and gu must be row-major and of one dtype")
    _lib.call(
        "nmb_gemm_bf16_swiglu_bwd", 1, m, f, h, dy.data_ptr(), max(dy.stride(0), h), wd.data_ptr(),
        max(wd.stride(0), f), gu.data_ptr(), gu.stride(0), dgu.data_ptr(), dgu.stride(0), _lib.ptr(out),
        out.stride(0) if out is not None else 0, _lib.stream_of(dy),
    )
    return dgu, out


def mm_gate_up_swiglu_bwd(a: Tensor, w_gu: Tensor, dy: Tensor, wd: Tensor, *, act: bool = True
                          ) -> tuple[Tensor, Tensor | None]:
    """The MLP backward of a recomputed block in one pass: the gate/up product
    ``[g|u] = a [Wg; Wu]^T`` (``w_gu`` [2F, K], as ``mm_gate_up`` computes it),
    ``ds = dy @ wd`` and the SwiGLU backward, for each tile of the output with
    g, u and ds in registers (``nmb_gemm_bf16_gate_up_swiglu_bwd``): the same
    (``dgu`` [M, 2F], ``silu(g) * u`` [M, F] if act) as ``mm_gate_up`` (product
    only) then ``mm_swiglu_bwd``, bit for bit, without [g|u] in memory.  Other
    dtypes run those two."""
    m, k = a.shape
    f2, k2 = w_gu.shape
    m2, h = dy.shape
    h2, f = wd.shape
    if k != k2 or f2 != 2 * f or m2 != m or h2 != h:
        raise ValueError("mm_gate_up_swiglu_bwd: a [M, K], w_gu [2F, K], dy [M, H] and wd [H, F] expected")
    if a.dtype != torch.bfloat16:
        _, gu = mm_gate_up(a, w_gu, act=False, gu=True)
        return mm_swiglu_bwd(dy, wd, gu, act=act)
    _require_gpu(a, w_gu, dy, wd)
    if any(t.stride(1) != 1 or t.dtype != a.dtype for t in (a, w_gu, dy, wd)):
        raise ValueError("mm_gate_up_swiglu_bwd: operands must be row-major and of one dtype")
    dgu = torch.empty(m, f2, dtype=a.dtype, device=a.device)
    out = torch.empty(m, f, dtype=a.dtype, device=a.device) if act else None
    _lib.call(
        "nmb_gemm_bf16_gate_up_swiglu_bwd", m, f, k, a.data_ptr(), max(a.stride(0), k), w_gu.data_ptr(),
        max(w_gu.stride(0), k), h, dy.data_ptr(), max(dy.stride(0), h), 1, wd.data_ptr(), max(wd.stride(0), f),
        dgu.data_ptr(), dgu.stride(0), _lib.ptr(out), out.stride(0) if out is not None else 0,
        _lib.stream_of(a),
    )
    return dgu, out


def mm_gate_up(a: Tensor, w_gu: Tensor, *, act: bool = True, gu: bool = False,
               act_out: Tensor | None = None, gu_out: Tensor | None = None
               ) -> tuple[Tensor | None, Tensor | None]:
    """The gate/up projections of GPTMLP.forward (models/gpt/mlp.py:72-78) with
    ``w_gu`` = [Wg; Wu] ([2F, K], row-major): returns (``silu(a Wg^T) * (a Wu^T)``
    if act, the product ``a [Wg; Wu]^T`` [M, 2F] if gu).  bf16 runs one GEMM
    with the activation as its epilogue (``nmb_gemm_bf16_swiglu``: one plan per
    shape, so the product is the same bits with or without the activation, and
    the activation equals ``swiglu_fwd`` of it); other dtypes run the GEMM and
    then ``swiglu_fwd``."""
    if not (act or gu):
        raise ValueError("mm_gate_up: nothing requested")
    m, k = a.shape
    f2, k2 = w_gu.shape
    if k != k2 or f2 % 2:
        raise ValueError("mm_gate_up: w_gu must be [2F, K] with a = [M, K]")
    f = f2 // 2
    if a.dtype != torch.bfloat16:
        p = mm(a, w_gu.t(), out=gu_out)
        s = swiglu_fwd(p[:, :f], p[:, f:], out=act_out) if act else None
        return s, (p if gu else None)
    _require_gpu(a, w_gu)
    if a.stride(1) != 1 or w_gu.stride(1) != 1 or w_gu.dtype != a.dtype:
        raise ValueError("mm_gate_up: a and w_gu must be row-major and of one dtype")
    s = p = None
    if act:
        s = act_out if act_out is not None else torch.empty(m, f, dtype=a.dtype, device=a.device)
        if s.shape != (m, f) or s.dtype != a.dtype or s.stride(1) != 1:
            raise ValueError("mm_gate_up: act_out must be a row-major [M, F] tensor of a's dtype")
    if gu:
        p = gu_out if gu_out is not None else torch.empty(m, f2, dtype=a.dtype, device=a.device)
        if p.shape != (m, f2) or p.dtype != a.dtype or p.stride(1) != 1:
            raise ValueError("mm_gate_up: gu_out must be a row-major [M, 2F] tensor of a's dtype")
    _lib.call(
        "nmb_gemm_bf16_swiglu", m, f, k, a.data_ptr(), max(a.stride(0), k), w_gu.data_ptr(),
        max(w_gu.stride(0), k), _lib.ptr(s), s.stride(0) if s is not None else 0, _lib.ptr(p),
        p.stride(0) if p is not None else 0, _lib.stream_of(a),
    )
    return s, p


def mm_swiglu(a: Tensor, w_gu: Tensor, out: Tensor | None = None) -> Tensor:
    """``silu(a Wg^T) * (a Wu^T)`` with ``w_gu`` = [Wg; Wu] (see ``mm_gate_up``)."""
    return mm_gate_up(a, w_gu, act=True, act_out=out)[0]


def swiglu_bwd(
    g: Tensor, u: Tensor, dout: Tensor, dg: Tensor, du: Tensor, out: Tensor | None = None
) -> None:
    _require_gpu(g, u, dout, dg, du)
    rows, cols = g.shape
    _lib.call(
        "nmb_swiglu_bwd", g.data_ptr(), g.stride(0), u.data_ptr(), u.stride(0), dout.data_ptr(),
        dout.stride(0), dg.data_ptr(), dg.stride(0), du.data_ptr(), du.stride(0),
        _lib.ptr(out), out.stride(0) if out is not None else cols, rows, cols,
        _lib.dtype_code(g.dtype), _lib.stream_of(g),
    )


class SwiGLUFunction(torch.autograd.Function):
    """``silu(gate) * up`` (models/gpt/mlp.py:77)."""

    @staticmethod
    def forward(ctx: Any, gate: Tensor, up: Tensor) -> Tensor:
        if gate.shape != up.shape:
            raise ValueError("gate and up must have the same shape")
        shape = gate.shape
        g2 = gate.reshape(-1, shape[-1]).contiguous()
        u2 = up.reshape(-1, shape[-1]).contiguous()
        out = swiglu_fwd(g2, u2)
        ctx.save_for_backward(g2, u2)
        ctx.shape = shape
        return out.view(shape)

    @staticmethod
    def backward(ctx: Any, grad: Tensor):
        g2, u2 = ctx.saved_tensors
        d2 = grad.reshape(g2.shape).contiguous()
        dg = torch.empty_like(g2)
        du = torch.empty_like(u2)
        swiglu_bwd(g2, u2, d2, dg, du)
        return dg.view(ctx.shape), du.view(ctx.shape)


def swiglu(gate: Tensor, up: Tensor) -> Tensor:
    require_precision(gate, up)
    return SwiGLUFunction.apply(gate, up)


# ---------------------------------------------------------------- attention
def _check_attn(q: Tensor, ks: Sequence[Tensor], vs: Sequence[Tensor]) -> tuple[int, ...]:
    require_precision(q, *ks, *vs)
    if q.ndim != 4 or any(k.ndim != 4 for k in ks) or any(v.ndim != 4 for v in vs):
        raise ValueError("q, k and v must have [batch, heads, sequence, head_dim] shape")
    for k, v in zip(ks, vs):
        if k.shape != v.shape:
            raise ValueError("k and v must have identical shapes")
        if k.shape != ks[0].shape:
            raise ValueError("all K/V blocks must have the same shape")
    k = ks[0]
    if q.shape[0] != k.shape[0] or q.shape[-1] != k.shape[-1]:
        raise ValueError("q and k/v must agree on batch size and head_dim")
    if q.shape[1] % k.shape[1]:
        raise ValueError(f"query heads ({q.shape[1]}) must be divisible by KV heads ({k.shape[1]})")
    return q.shape[0], q.shape[1], k.shape[1], q.shape[2], k.shape[2], q.shape[3]


def attn_fwd_bshd(
    q: Tensor,
    ks: Sequence[Tensor],
    vs: Sequence[Tensor],
    k_offsets: Sequence[int],
    *,
    causal: bool,
    q_offset: int,
    scale: float | None,
    out: Tensor | None = None,
    lse: Tensor | None = None,
) -> tuple[Tensor, Tensor]:
    """Attention over [B,S,H,D]-strided q and K/V blocks; returns (o [B,S,Hq,D], lse [B,Hq,S])."""
    _require_gpu(q, *ks, *vs)
    b, sq, hq, d = q.shape
    _, sk, hkv, _ = ks[0].shape
    if out is None:
        out = torch.empty(b, sq, hq, d, dtype=q.dtype, device=q.device)
    if lse is None:
        lse = torch.empty(b, hq, sq, dtype=torch.float32, device=q.device)
    kv_strides = _eff_strides(ks[0])
    for t in (*ks, *vs):
        if _eff_strides(t) != kv_strides or t.stride(3) != 1:
            raise ValueError("attention: all K/V blocks must share one [B,S,H,D] stride layout")
    if q.stride(3) != 1 or out.stride(3) != 1:
        raise ValueError("attention: head_dim must be the contiguous dimension")
    _lib.call(
        "nmb_attn_fwd", q.data_ptr(), _lib.ptr_array(k.data_ptr() for k in ks),
        _lib.ptr_array(v.data_ptr() for v in vs), _lib.i64_array(k_offsets), len(ks),
        out.data_ptr(), lse.data_ptr(), b, hq, hkv, sq, sk, d,
        _lib.i64x3(_eff_strides(q)), _lib.i64x3(kv_strides), _lib.i64x3(_eff_strides(out)),
        1 if causal else 0, int(q_offset), float(scale) if scale else 0.0,
        _lib.dtype_code(q.dtype), _lib.stream_of(q),
    )
    return out, lse


def attn_fwd_from_lse_bshd(q: Tensor, ks: Sequence[Tensor], vs: Sequence[Tensor],
                           k_offsets: Sequence[int], lse: Tensor, *, causal: bool, q_offset: int,
                           scale: float | None, out: Tensor | None = None) -> Tensor:
    """The attention output recomputed from a saved lse [B,Hq,S] (bf16):
    P = exp(S - lse) without the online max/rescale; equal to attn_fwd_bshd's
    output within bf16 rounding."""
    _require_gpu(q, *ks, *vs, lse)
    b, sq, hq, d = q.shape
    _, sk, hkv, _ = ks[0].shape
    if out is None:
        out = torch.empty(b, sq, hq, d, dtype=q.dtype, device=q.device)
    if lse.shape != (b, hq, sq) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError("attention: lse must be a contiguous fp32 [B, Hq, S] tensor")
    kv_strides = _eff_strides(ks[0])
    for t in (*ks, *vs):
        if _eff_strides(t) != kv_strides or t.stride(3) != 1:
            raise ValueError("attention: all K/V blocks must share one [B,S,H,D] stride layout")
    if q.stride(3) != 1 or out.stride(3) != 1:
        raise ValueError("attention: head_dim must be the contiguous dimension")
    _lib.call(
        "nmb_attn_fwd_from_lse", q.data_ptr(), _lib.ptr_array(k.data_ptr() for k in ks),
        _lib.ptr_array(v.data_ptr() for v in vs), _lib.i64_array(k_offsets), len(ks),
        lse.data_ptr(), out.data_ptr(), b, hq, hkv, sq, sk, d,
        _lib.i64x3(_eff_strides(q)), _lib.i64x3(kv_strides), _lib.i64x3(_eff_strides(out)),
        1 if causal else 0, int(q_offset), float(scale) if scale else 0.0,
        _lib.dtype_code(q.dtype), _lib.stream_of(q),
    )
    return out


def attn_bwd_bshd(
    q: Tensor,
    ks: Sequence[Tensor],
    vs: Sequence[Tensor],
    k_offsets: Sequence[int],
    o: Tensor,
    do: Tensor,
    lse: Tensor,
    dq: Tensor,
    dks: Sequence[Tensor],
    dvs: Sequence[Tensor],
    *,
    causal: bool,
    q_offset: int,
    scale: float | None,
) -> None:
    """Backward of attn_fwd_bshd into caller-provided dq / dK / dV (same strides as q / K / V)."""
    _require_gpu(q, o, do, lse, dq)
    b, sq, hq, d = q.shape
    _, sk, hkv, _ = ks[0].shape
    kv_strides = _eff_strides(ks[0])
    for t in (*ks, *vs, *dks, *dvs):
        if _eff_strides(t) != kv_strides or t.stride(3) != 1:
            raise ValueError("attention backward: K, V, dK, dV must share one stride layout")
    if _eff_strides(dq) != _eff_strides(q) or _eff_strides(do) != _eff_strides(o):
        raise ValueError("attention backward: dq must match q's strides and dO must match O's")
    nbytes = _lib.ctypes.c_size_t(0)
    _lib.call("nmb_attn_bwd_workspace_bytes", b, hq, sq, _lib.ctypes.byref(nbytes))
    ws = _workspace(nbytes.value, q.device)
    _lib.call(
        "nmb_attn_bwd", q.data_ptr(), _lib.ptr_array(k.data_ptr() for k in ks),
        _lib.ptr_array(v.data_ptr() for v in vs), _lib.i64_array(k_offsets), len(ks),
        o.data_ptr(), do.data_ptr(), lse.data_ptr(), dq.data_ptr(),
        _lib.ptr_array(t.data_ptr() for t in dks), _lib.ptr_array(t.data_ptr() for t in dvs),
        ws.data_ptr(), ws.numel(), b, hq, hkv, sq, sk, d,
        _lib.i64x3(_eff_strides(q)), _lib.i64x3(kv_strides), _lib.i64x3(_eff_strides(o)),
        1 if causal else 0, int(q_offset), float(scale) if scale else 0.0,
        _lib.dtype_code(q.dtype), _lib.stream_of(q),
    )


def attn_bwd_rope_bshd(q: Tensor, k: Tensor, v: Tensor, o: Tensor, do: Tensor, lse: Tensor,
                       dq: Tensor, dk: Tensor, dv: Tensor, *, causal: bool, q_offset: int,
                       scale: float | None, cos: Tensor, sin: Tensor, pos_offset: int = 0,
                       positions: Tensor | None = None) -> None:
    """attn_bwd_bshd of one K/V block (self-attention of the local sequence) with the
    RoPE backward of q and k fused into the dq / dk stores: dq and dk come out
    rotated by -theta, as attn_bwd_bshd followed by rope_apply(inverse=True)."""
    if q.dtype != torch.bfloat16 or q.shape[3] not in (64, 128):
        attn_bwd_bshd(q, [k], [v], (0,), o, do, lse, dq, [dk], [dv], causal=causal,
                      q_offset=q_offset, scale=scale)
        rope_apply(dq, dq, cos, sin, pos_offset=pos_offset, positions=positions, inverse=True)
        rope_apply(dk, dk, cos, sin, pos_offset=pos_offset, positions=positions, inverse=True)
        return
    _require_gpu(q, o, do, lse, dq, cos, sin)
    b, s, hq, d = q.shape
    hkv = k.shape[2]
    kv_strides = _eff_strides(k)
    for t in (v, dk, dv):
        if _eff_strides(t) != kv_strides or t.stride(3) != 1:
            raise ValueError("attention backward: K, V, dK, dV must share one stride layout")
    if _eff_strides(dq) != _eff_strides(q) or _eff_strides(do) != _eff_strides(o):
        raise ValueError("attention backward: dq must match q's strides and dO must match O's")
    pos_ptr, pos_bstride = None, 0
    if positions is not None:
        if positions.dtype != torch.int32:
            raise ValueError("attention backward: positions must be int32")
        pos_ptr = positions.data_ptr()
        pos_bstride = positions.stride(0) if positions.ndim == 2 else 0
    nbytes = _lib.ctypes.c_size_t(0)
    _lib.call("nmb_attn_bwd_workspace_bytes", b, hq, s, _lib.ctypes.byref(nbytes))
    ws = _workspace(nbytes.value, q.device)
    _lib.call(
        "nmb_attn_bwd_rope", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
        lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws.numel(),
        b, hq, hkv, s, d, _lib.i64x3(_eff_strides(q)), _lib.i64x3(kv_strides),
        _lib.i64x3(_eff_strides(o)), 1 if causal else 0, int(q_offset),
        float(scale) if scale else 0.0, cos.data_ptr(), sin.data_ptr(), cos.shape[0], pos_ptr,
        pos_bstride, int(pos_offset), _lib.stream_of(q),
    )


class AttentionFunction(torch.autograd.Function):
    """Attention over K/V blocks for [B,H,S,D] tensors (views of [B,S,H,D] memory).

    One block with offset 0 is ``local_attention`` (nn/kernels/torch_backend.py:25-76,
    key positions arange(Sk), query positions sequence_offset + arange(Sq)); several
    blocks with absolute key offsets are one ring rank's share
    (context_parallel/ring.py:104-250).  Saves only q, K/V, the output and the lse.
    """

    @staticmethod
    def forward(ctx: Any, q: Tensor, causal: bool, q_offset: int, scale: float | None,
                k_offsets: tuple[int, ...], *kv: Tensor) -> Tensor:
        n = len(kv) // 2
        ks = [_canonical_bhsd(t) for t in kv[:n]]
        vs = [_canonical_bhsd(t) for t in kv[n:]]
        _check_attn(q, ks, vs)
        q = _canonical_bhsd(q)
        o, lse = attn_fwd_bshd(
            _bshd_view(q), [_bshd_view(k) for k in ks], [_bshd_view(v) for v in vs], k_offsets,
            causal=causal, q_offset=q_offset, scale=scale,
        )
        o_bhsd = o.transpose(1, 2)
        ctx.save_for_backward(q, o_bhsd, lse, *ks, *vs)
        ctx.meta = (causal, q_offset, scale, tuple(k_offsets), n)
        return o_bhsd

    @staticmethod
    def backward(ctx: Any, grad: Tensor):
        causal, q_offset, scale, k_offsets, n = ctx.meta
        q, o, lse, *kv = ctx.saved_tensors
        ks, vs = kv[:n], kv[n:]
        do = _canonical_bhsd(grad)
        dq = _new_bhsd(q.shape, q)
        dks = [_new_bhsd(k.shape, k) for k in ks]
        dvs = [_new_bhsd(v.shape, v) for v in vs]
        attn_bwd_bshd(
            _bshd_view(q), [_bshd_view(k) for k in ks], [_bshd_view(v) for v in vs], k_offsets,
            _bshd_view(o), _bshd_view(do), lse, _bshd_view(dq),
            [_bshd_view(t) for t in dks], [_bshd_view(t) for t in dvs],
            causal=causal, q_offset=q_offset, scale=scale,
        )
        return (dq, None, None, None, None, *dks, *dvs)


def attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    *,
    causal: bool = True,
    sequence_offset: int = 0,
    scale: float | None = None,
) -> Tensor:
    """``local_attention`` for [B,H,S,D] tensors, GQA without repeated K/V.
    The bf16 MFMA kernels take heads of 64 and 128; smaller bf16 heads run on
    them zero-padded to the next of the two (the padded dimensions add zero to
    every score and give zero output columns, which are cut off; the scale
    stays 1/sqrt(D) of the true size), and autograd pads and cuts the
    gradients the same way."""
    _check_attn(q, [k], [v])
    d = q.shape[-1]
    if q.dtype == torch.bfloat16 and d not in (64, 128) and d < 128:
        dp = 64 if d < 64 else 128
        scale = scale if scale else 1.0 / math.sqrt(d)
        qp, kp, vp = (torch.nn.functional.pad(t, (0, dp - d)) for t in (q, k, v))
        return AttentionFunction.apply(qp, causal, int(sequence_offset), scale, (0,), kp, vp)[..., :d]
    return AttentionFunction.apply(q, causal, int(sequence_offset), scale, (0,), k, v)


def _mask_args(mask: Tensor, q: Tensor, shape: tuple[int, int, int, int]) -> tuple[Tensor, int, tuple]:
    """(mask tensor, kind, element strides over [B, Hq, Sq, Sk]) of an SDPA
    attn_mask: broadcast like SDPA's (trailing dimensions), 0 strides where it
    broadcasts; kind 1 boolean, 2 additive in q's dtype."""
    if mask.dtype == torch.bool:
        kind = 1
    elif mask.dtype == q.dtype:
        kind = 2
    else:
        raise ValueError(f"attention_mask must be boolean or of the query dtype {q.dtype}, got {mask.dtype}")
    if mask.device != q.device:
        raise ValueError("attention_mask must be on the query's device")
    try:
        full = torch.broadcast_to(mask, shape)
    except RuntimeError as exc:
        raise ValueError(f"attention_mask of shape {tuple(mask.shape)} does not broadcast to {shape}") from exc
    return mask, kind, tuple(st if n > 1 else 0 for st, n in zip(full.stride(), shape))


class MaskedAttentionFunction(torch.autograd.Function):
    """``local_attention`` with ``attention_mask`` and/or ``dropout_p``
    (nn/kernels/torch_backend.py:60-76): the mask ANDed with the causal mask
    (boolean masks) or added to the scores (masks of the query dtype), one K/V
    block; dropout of the normalised probabilities with the counter-based mask
    of ``seed``; ``nmb_attn_masked_*``.  The mask itself gets no gradient."""

    @staticmethod
    def forward(ctx: Any, q: Tensor, k: Tensor, v: Tensor, mask: Tensor | None, causal: bool,
                q_offset: int, scale: float | None, dropout_p: float, seed: int) -> Tensor:
        b, hq, hkv, sq, sk, d = _check_attn(q, [k], [v])
        q, k, v = (_canonical_bhsd(t) for t in (q, k, v))
        if mask is None:
            kind, mstrides = 0, (0, 0, 0, 0)
        else:
            mask, kind, mstrides = _mask_args(mask, q, (b, hq, sq, sk))
        mask_ptr = mask.data_ptr() if mask is not None else None
        o = _new_bhsd(q.shape, q)
        lse = torch.empty(b, hq, sq, dtype=torch.float32, device=q.device)
        qs, ks, os_ = (_eff_strides(_bshd_view(t)) for t in (q, k, o))
        _lib.call(
            "nmb_attn_masked_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
            b, hq, hkv, sq, sk, d, _lib.i64x3(qs), _lib.i64x3(ks), _lib.i64x3(os_), mask_ptr, kind,
            _lib.i64_array(mstrides), 1 if causal else 0, int(q_offset), float(scale) if scale else 0.0,
            float(dropout_p), int(seed), _lib.dtype_code(q.dtype), _lib.stream_of(q),
        )
        ctx.save_for_backward(q, k, v, o, lse, mask)
        ctx.meta = (causal, q_offset, scale, kind, mstrides, dropout_p, seed)
        return o

    @staticmethod
    def backward(ctx: Any, grad: Tensor):
        causal, q_offset, scale, kind, mstrides, dropout_p, seed = ctx.meta
        q, k, v, o, lse, mask = ctx.saved_tensors
        b, hq, sq, d = q.shape
        hkv, sk = k.shape[1], k.shape[2]
        do = _canonical_bhsd(grad)
        dq, dk, dv = _new_bhsd(q.shape, q), _new_bhsd(k.shape, k), _new_bhsd(v.shape, v)
        nbytes = _lib.ctypes.c_size_t(0)
        _lib.call("nmb_attn_bwd_workspace_bytes", b, hq, sq, _lib.ctypes.byref(nbytes))
        ws = _workspace(nbytes.value, q.device)
        if _eff_strides(_bshd_view(do)) != _eff_strides(_bshd_view(o)):
            do = _canonical_bhsd(do.contiguous())
        _lib.call(
            "nmb_attn_masked_bwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
            lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws.numel(),
            b, hq, hkv, sq, sk, d, _lib.i64x3(_eff_strides(_bshd_view(q))),
            _lib.i64x3(_eff_strides(_bshd_view(k))), _lib.i64x3(_eff_strides(_bshd_view(o))),
            mask.data_ptr() if mask is not None else None, kind, _lib.i64_array(mstrides),
            1 if causal else 0, int(q_offset), float(scale) if scale else 0.0, float(dropout_p), int(seed),
            _lib.dtype_code(q.dtype), _lib.stream_of(q),
        )
        return dq, dk, dv, None, None, None, None, None, None


def _check_dropout_p(p: float) -> float:
    p = float(p)
    if not 0.0 <= p < 1.0:
        raise ValueError(f"dropout probability must be in [0, 1), got {p}")
    return p


def dropout_seed() -> int:
    """A 63-bit key for the counter-based dropout masks, drawn from torch's
    default CPU generator, so that whatever replays that generator replays the
    mask: the recompute of a torch activation checkpoint (preserve_rng_state)
    and a forked, explicitly seeded stream (nn.activation_rng_context).  Each
    draw advances that CPU generator, where the reference's F.dropout on the
    GPU advances the CUDA generator instead: without an rng fork around the
    dropout, later CPU randomness (data shuffles, initialisation) differs from
    a reference run with the same seed."""
    return int(torch.randint(0, 2**63 - 1, (1,), dtype=torch.int64).item())


def masked_attention(q: Tensor, k: Tensor, v: Tensor, attention_mask: Tensor | None, *,
                     causal: bool = True, sequence_offset: int = 0, scale: float | None = None,
                     dropout_p: float = 0.0, seed: int | None = None) -> Tensor:
    """``local_attention`` with ``attention_mask`` and/or ``dropout_p`` for
    [B,H,S,D] tensors; ``seed`` keys the dropout mask (default: dropout_seed())."""
    dropout_p = _check_dropout_p(dropout_p)
    _require_gpu(q, k, v, attention_mask)
    require_precision(q, k, v)
    if causal and attention_mask is not None and attention_mask.dtype != torch.bool:
        # the reference combines the masks with `mask & causal_mask` (torch_backend.py:66)
        raise ValueError("a causal attention_mask must be boolean (it is ANDed with the causal mask)")
    if dropout_p and seed is None:
        seed = dropout_seed()
    return MaskedAttentionFunction.apply(q, k, v, attention_mask, bool(causal), int(sequence_offset), scale,
                                         dropout_p, int(seed or 0))


def ring_attention(
    q: Tensor,
    kv_blocks: Sequence[tuple[Tensor, Tensor]],
    key_offsets: Sequence[int],
    *,
    causal: bool = True,
    query_offset: int = 0,
    scale: float | None = None,
) -> Tensor:
    """One context-parallel rank's attention over streamed K/V blocks, merged by
    online softmax in one kernel (context_parallel/ring.py:104-250 on one GPU)."""
    if not 1 <= len(kv_blocks) <= 8:
        raise ValueError("ring_attention supports 1 to 8 K/V blocks")
    ks = [k for k, _ in kv_blocks]
    vs = [v for _, v in kv_blocks]
    _check_attn(q, ks, vs)
    return AttentionFunction.apply(
        q, causal, int(query_offset), scale, tuple(int(o) for o in key_offsets), *ks, *vs
    )


# ---------------------------------------------------------------- dropout
class DropoutAddFunction(torch.autograd.Function):
    """``residual + F.dropout(x, p)`` (models/gpt/layer.py:114-137, nn/dropout.py:
    47-70) as one ``nmb_dropout_add`` pass, residual optional; the backward is
    the same kernel on the gradient with the same seed (the mask is a function
    of (seed, element index), nothing is saved)."""

    @staticmethod
    def forward(ctx: Any, x: Tensor, residual: Tensor | None, p: float, seed: int) -> Tensor:
        xc = x.contiguous()
        rc = residual.contiguous() if residual is not None else None
        out = torch.empty_like(xc)
        _lib.call("nmb_dropout_add", xc.data_ptr(), rc.data_ptr() if rc is not None else None,
                  out.data_ptr(), xc.numel(), p, seed, _lib.dtype_code(x.dtype), _lib.stream_of(x))
        ctx.meta = (p, seed, residual is not None)
        return out

    @staticmethod
    def backward(ctx: Any, grad: Tensor):
        p, seed, has_residual = ctx.meta
        g = grad.contiguous()
        dx = torch.empty_like(g)
        _lib.call("nmb_dropout_add", g.data_ptr(), None, dx.data_ptr(), g.numel(), p, seed,
                  _lib.dtype_code(g.dtype), _lib.stream_of(g))
        return dx, (grad if has_residual else None), None, None


def dropout_add(x: Tensor, p: float, *, seed: int | None = None, residual: Tensor | None = None) -> Tensor:
    """``residual + dropout(x, p)`` (just the dropout without ``residual``) in the
    training mode of F.dropout: kept elements scaled by 1 / (1 - p); ``seed``
    keys the mask (default: dropout_seed())."""
    p = _check_dropout_p(p)
    _require_gpu(x, residual)
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype
                                 or residual.device != x.device):
        raise ValueError(
            f"residual {tuple(residual.shape)} {residual.dtype} does not match x {tuple(x.shape)} {x.dtype}"
        )
    if seed is None:
        seed = dropout_seed()
    return DropoutAddFunction.apply(x, residual, p, int(seed))


# ---------------------------------------------------------------- LM head + CE
def _padded_head(weight: Tensor) -> tuple[Tensor, int]:
    """The LM-head table with its vocabulary rows zero-padded to a multiple of
    8 (the GEMM and cross-entropy kernels move 16-byte chunks), and the true
    vocabulary size; the table itself when no padding is needed."""
    vocab = weight.shape[0]
    if vocab % 8 == 0:
        return weight, vocab
    return _zero_padded(weight, _round8(vocab), weight.shape[1]), vocab


def _mask_padding(logits: Tensor, vocab: int) -> None:
    """-inf in the padded vocabulary columns: they add exp(-inf) = 0 to the
    softmax and get a zero gradient."""
    if logits.shape[1] > vocab:
        logits[:, vocab:].fill_(float("-inf"))


def ce_fwd(logits2: Tensor, targets: Tensor, ignore_index: int, loss: Tensor, lse: Tensor) -> None:
    rows, vocab = logits2.shape
    _lib.call(
        "nmb_ce_fwd", logits2.data_ptr(), logits2.stride(0), targets.data_ptr(), rows, vocab,
        int(ignore_index), loss.data_ptr(), lse.data_ptr(), _lib.dtype_code(logits2.dtype),
        _lib.stream_of(logits2),
    )


def ce_bwd_(logits2: Tensor, targets: Tensor, ignore_index: int, lse: Tensor, grad: Tensor) -> None:
    rows, vocab = logits2.shape
    _lib.call(
        "nmb_ce_bwd", logits2.data_ptr(), logits2.stride(0), targets.data_ptr(), rows, vocab,
        int(ignore_index), lse.data_ptr(), grad.data_ptr(), _lib.dtype_code(logits2.dtype),
        _lib.stream_of(logits2),
    )


def _chunks(rows: int, chunk: int):
    for start in range(0, rows, chunk):
        yield start, min(rows, start + chunk)


# ---------------------------------------------------------------- embedding
class TiedGrad:
    """Hands the tied LM head's table gradient to the embedding's backward,
    which adds it to its own in the same pass (models/gpt/model.py:125-142:
    one weight shared by VocabParallelEmbedding and VocabParallelLinear).  The
    LM head's backward always runs first: the embedding output feeds every
    layer before the head."""

    __slots__ = ("grad",)

    def __init__(self) -> None:
        self.grad: Tensor | None = None


class EmbeddingFunction(torch.autograd.Function):
    """Row gather of the [V, H] table (tensor_parallel/embedding.py:60-74 at TP=1)
    and its deterministic scatter-add backward, merged with the tied LM-head
    gradient when a ``TiedGrad`` carries it."""

    @staticmethod
    def forward(ctx: Any, weight: Tensor, ids: Tensor, tie: TiedGrad | None) -> Tensor:
        _require_gpu(weight, ids)
        vocab, hidden = weight.shape
        out = torch.empty(*ids.shape, hidden, dtype=weight.dtype, device=weight.device)
        _lib.call("nmb_embedding_fwd", weight.data_ptr(), ids.data_ptr(), out.data_ptr(), ids.numel(),
                  vocab, hidden, _lib.dtype_code(weight.dtype), _lib.stream_of(weight))
        ctx.save_for_backward(ids)
        ctx.shape = (vocab, hidden, weight.dtype)
        ctx.tie = tie
        return out

    @staticmethod
    def backward(ctx: Any, dout: Tensor):
        (ids,) = ctx.saved_tensors
        vocab, hidden, dtype = ctx.shape
        dout = dout.to(dtype).contiguous()
        grad_in = None
        if ctx.tie is not None:
            grad_in, ctx.tie.grad = ctx.tie.grad, None
        grad = torch.empty(vocab, hidden, dtype=dtype, device=dout.device)
        _lib.call("nmb_embedding_bwd", dout.data_ptr(), ids.data_ptr(), _lib.ptr(grad_in), grad.data_ptr(),
                  ids.numel(), vocab, hidden, _lib.dtype_code(dtype), _lib.stream_of(dout))
        return grad, None, None


def embedding(weight: Tensor, ids: Tensor, tie: TiedGrad | None = None) -> Tensor:
    """VocabParallelEmbedding's lookup at TP=1 on the GPU kernels
    (tensor_parallel/embedding.py:60-68): ``F.embedding(ids, weight)`` for ids in
    [0, V); an id outside the table gives a zero row and no table gradient."""
    if ids.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"input_ids must be an integer tensor, got {ids.dtype}")
    return EmbeddingFunction.apply(weight, ids.to(torch.int64).contiguous(), tie)


class LMHeadCrossEntropyFunction(torch.autograd.Function):
    """Tied LM head + token cross entropy without full logits.

    Forward, per token chunk: logits = x_c E^T (one GEMM into a [chunk, V]
    buffer), then ``nmb_ce_fwd`` -> per-token loss and lse.  Only lse is kept.
    Backward, per chunk: recompute the chunk's logits, ``nmb_ce_bwd`` turns them
    in place into G = (softmax - onehot) * grad, then dx_c = G E and
    dE += G^T x_c (fixed chunk order: deterministic), summed in fp32 and rounded
    to bf16 once, as the reference's single product G^T X is.  Matches
    VocabParallelLinear + _VocabParallelCrossEntropy at TP=1
    (tensor_parallel/layers.py:207-214, cross_entropy.py:30-86).
    """

    @staticmethod
    def forward(ctx: Any, x2: Tensor, weight: Tensor, targets: Tensor, ignore_index: int,
                chunk: int, tie: TiedGrad | None = None) -> Tensor:
        _require_gpu(x2, weight, targets)
        rows = x2.shape[0]
        loss = torch.empty(rows, dtype=torch.float32, device=x2.device)
        lse = torch.empty_like(loss)
        w, vocab = _padded_head(weight)
        buf = torch.empty(min(chunk, max(rows, 1)), w.shape[0], dtype=x2.dtype, device=x2.device)
        for s, e in _chunks(rows, chunk):
            logits = buf[: e - s]
            mm(x2[s:e], w.t(), out=logits)
            _mask_padding(logits, vocab)
            ce_fwd(logits, targets[s:e], ignore_index, loss[s:e], lse[s:e])
        ctx.save_for_backward(x2, weight, targets, lse)
        ctx.ignore_index = ignore_index
        ctx.chunk = chunk
        ctx.tie = tie
        return loss

    @staticmethod
    def backward(ctx: Any, grad_loss: Tensor):
        x2, weight, targets, lse = ctx.saved_tensors
        grad_loss = grad_loss.float().contiguous()
        rows = x2.shape[0]
        dx = torch.empty_like(x2)
        f32 = weight.dtype == torch.float32
        w, vocab = _padded_head(weight)
        # the bf16 gradient accumulates over the chunks in fp32 (one rounding at the end)
        if f32:
            dw = torch.zeros_like(w)
        else:  # the first chunk writes it (beta 0)
            dw = (torch.empty if rows > 0 else torch.zeros)(w.shape, dtype=torch.float32,
                                                             device=weight.device)
        buf = torch.empty(min(ctx.chunk, max(rows, 1)), w.shape[0], dtype=x2.dtype,
                          device=x2.device)
        for i, (s, e) in enumerate(_chunks(rows, ctx.chunk)):
            g = buf[: e - s]
            mm(x2[s:e], w.t(), out=g)
            _mask_padding(g, vocab)
            ce_bwd_(g, targets[s:e], ctx.ignore_index, lse[s:e], grad_loss[s:e])
            mm(g, w, out=dx[s:e])
            if f32:
                mm(g.t(), x2[s:e], out=dw, c=dw, beta=1.0)
            else:
                mm_f32out(g.t(), x2[s:e], dw, beta=0.0 if i == 0 else 1.0)
        dw = dw[:vocab]
        if not f32:
            dw = dw.to(weight.dtype)
        if ctx.tie is not None:  # the embedding's backward adds it to its own gradient
            ctx.tie.grad = dw
            return dx, None, None, None, None, None
        return dx, dw, None, None, None, None


class TargetCheck:
    """The cross entropy's target-range check (tensor_parallel/cross_entropy.py:
    109-114: a ValueError for ids outside [0, vocab) other than ignore_index),
    enqueued when constructed: the flag ``any(invalid)`` is copied to pinned
    host memory behind an event.  ``raise_if_invalid`` waits for that event
    only, so a check made at the start of the forward costs the host no wait
    for the layers enqueued after it (as ``torch.any`` at the loss would)."""

    def __init__(self, targets: Tensor, vocab: int, ignore_index: int = IGNORE_INDEX) -> None:
        invalid = (targets != ignore_index) & ((targets < 0) | (targets >= vocab))
        self._bad: bool | None = None
        if targets.device.type == "cuda":
            self._flag = torch.empty((), dtype=torch.bool, pin_memory=True)
            self._flag.copy_(invalid.any(), non_blocking=True)
            self._event = torch.cuda.Event()
            self._event.record(torch.cuda.current_stream(targets.device))
        else:
            self._bad = bool(invalid.any())

    def raise_if_invalid(self) -> None:
        if self._bad is None:
            self._event.synchronize()
            self._bad = bool(self._flag)
        if self._bad:
            raise ValueError("targets contain ids outside the original (unpadded) vocabulary")


def lm_head_cross_entropy(
    hidden: Tensor,
    weight: Tensor,
    targets: Tensor,
    *,
    ignore_index: int = IGNORE_INDEX,
    reduction: str = "mean",
    chunk: int = 2048,
    validate: "bool | TargetCheck" = True,
    tie: TiedGrad | None = None,
) -> Tensor:
    """Loss of ``F.linear(hidden, weight)`` under VocabParallelCrossEntropy
    (tensor_parallel/cross_entropy.py:89-123) without materialising logits."""
    if reduction not in ("none", "mean", "sum"):
        raise ValueError(f"unsupported reduction: {reduction}")
    require_precision(hidden, weight)
    if hidden.shape[:-1] != targets.shape:
        raise ValueError(
            "targets must match all non-vocabulary logits dimensions: "
            f"hidden={tuple(hidden.shape)}, targets={tuple(targets.shape)}"
        )
    vocab = weight.shape[0]
    if isinstance(validate, TargetCheck):
        validate.raise_if_invalid()
    elif validate:
        TargetCheck(targets, vocab, ignore_index).raise_if_invalid()
    x2 = hidden.reshape(-1, hidden.shape[-1]).contiguous()
    t1 = targets.reshape(-1).to(torch.int64).contiguous()
    loss = LMHeadCrossEntropyFunction.apply(x2, weight, t1, int(ignore_index), int(chunk), tie)
    if reduction == "none":
        return loss.view(targets.shape)
    if reduction == "sum":
        return loss.sum()
    valid = (t1 != ignore_index).sum().clamp_min(1)
    return loss.sum() / valid
