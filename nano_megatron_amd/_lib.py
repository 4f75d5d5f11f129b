"""ctypes binding of libnmb.so (declared in include/nmb.h).

The library is loaded once per process from this package directory.  There is
no CPU fallback: if the library is missing or cannot be loaded, every op
raises.  PyTorch supplies device memory and the current HIP stream; the
library shares torch's HIP runtime (one runtime per process).
"""

from __future__ import annotations

import ctypes
import pathlib
import threading

import torch

LIB_PATH = pathlib.Path(__file__).resolve().with_name("libnmb.so")

NMB_OK = 0
NMB_EINVAL = 1
NMB_EUNSUPPORTED = 2
NMB_EHIP = 3

NMB_F32 = 0
NMB_BF16 = 1

# nmb_abi_version() of the sources these signatures follow
ABI_VERSION = 2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_u64 = ctypes.c_uint64
_sz = ctypes.c_size_t
_pi64 = ctypes.POINTER(ctypes.c_int64)
_psz = ctypes.POINTER(ctypes.c_size_t)

# name -> argtypes (every function returns int status unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "nmb_last_error": [],
    "nmb_abi_version": [],
    "nmb_rmsnorm_fwd": [_p, _p, _p, _p, _i64, _i64, _f32, _i32, _p],
    "nmb_rmsnorm_bwd_workspace_bytes": [_i64, _i64, _psz],
    "nmb_rmsnorm_bwd": [_p, _p, _p, _p, _p, _p, _p, _sz, _i64, _i64, _f32, _i32, _p],
    "nmb_rmsnorm_bwd_rows": [_p, _p, _p, _p, _p, _p, _sz, _i64, _i64, _f32, _i32, _p],
    "nmb_rmsnorm_bwd_dw": [_p, _sz, _i64, _i64, _p, _i32, _p],
    "nmb_rope_table": [_p, _p, _p, _i64, _i64, _p],
    "nmb_rope_apply": [
        _p, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _pi64, _pi64, _i32, _i32, _p,
    ],
    "nmb_swiglu_fwd": [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i32, _p],
    "nmb_swiglu_bwd": [
        _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i32, _p,
    ],
    "nmb_attn_fwd": [
        _p, _p, _p, _pi64, _i32, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
        _pi64, _pi64, _pi64, _i32, _i64, _f32, _i32, _p,
    ],
    "nmb_attn_fwd_from_lse": [
        _p, _p, _p, _pi64, _i32, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
        _pi64, _pi64, _pi64, _i32, _i64, _f32, _i32, _p,
    ],
    "nmb_attn_bwd_workspace_bytes": [_i64, _i64, _i64, _psz],
    "nmb_attn_bwd": [
        _p, _p, _p, _pi64, _i32, _p, _p, _p, _p, _p, _p, _p, _sz, _i64, _i64, _i64, _i64, _i64,
        _i64, _pi64, _pi64, _pi64, _i32, _i64, _f32, _i32, _p,
    ],
    "nmb_attn_bwd_noalloc": [
        _p, _p, _p, _pi64, _i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
        _pi64, _pi64, _pi64, _i32, _i64, _f32, _i32, _p,
    ],
    "nmb_attn_bwd_rope": [
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _i64, _i64, _i64, _i64, _i64, _pi64, _pi64,
        _pi64, _i32, _i64, _f32, _p, _p, _i64, _p, _i64, _i64, _p,
    ],
    "nmb_attn_masked_fwd": [
        _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _pi64, _pi64, _pi64, _p, _i32,
        _pi64, _i32, _i64, _f32, _f32, _u64, _i32, _p,
    ],
    "nmb_attn_masked_bwd": [
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _i64, _i64, _i64, _i64, _i64, _i64, _pi64,
        _pi64, _pi64, _p, _i32, _pi64, _i32, _i64, _f32, _f32, _u64, _i32, _p,
    ],
    "nmb_dropout_add": [_p, _p, _p, _i64, _f32, _u64, _i32, _p],
    "nmb_embedding_fwd": [_p, _p, _p, _i64, _i64, _i64, _i32, _p],
    "nmb_embedding_bwd": [_p, _p, _p, _p, _i64, _i64, _i64, _i32, _p],
    "nmb_ce_fwd": [_p, _i64, _p, _i64, _i64, _i64, _p, _p, _i32, _p],
    "nmb_ce_bwd": [_p, _i64, _p, _i64, _i64, _i64, _p, _p, _i32, _p],
    "nmb_gemm_bf16_workspace_bytes": [_i32, _i32, _i64, _i64, _i64, _pi64],
    "nmb_gemm_bf16": [
        _i32, _i32, _i64, _i64, _i64, _f32, _p, _i64, _p, _i64, _f32, _p, _i64, _p, _i64, _p,
        _i64, _p,
    ],
    "nmb_gemm_f32": [
        _i32, _i32, _i64, _i64, _i64, _f32, _p, _i64, _p, _i64, _f32, _p, _i64, _p, _i64, _p,
    ],
    "nmb_gemm_bf16_f32out": [
        _i32, _i32, _i64, _i64, _i64, _f32, _p, _i64, _p, _i64, _f32, _p, _i64, _p, _i64, _p,
    ],
    "nmb_gemm_bf16_rope": [
        _i32, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64,
        _i64, _i64, _p,
    ],
    "nmb_gemm_bf16_swiglu": [_i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p],
    "nmb_gemm_bf16_swiglu_bwd": [_i32, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _p],
    "nmb_gemm_bf16_gate_up_swiglu_bwd": [_i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _i64, _i32, _p, _i64,
                                         _p, _i64, _p, _i64, _p],
    "nmb_adamw_workspace_bytes": [_i64, _psz],
    "nmb_adamw_step": [
        _p, _p, _p, _i32, _i64, _p, _p, _p, _i32, _i32, _f64, _f64, _f64, _f64, _f64, _i64, _f32,
        _p, _p, _sz, _p,
    ],
    "nmb_adamw_hyper_bytes": [_psz],
    "nmb_adamw_hyper": [_f64, _f64, _f64, _f64, _f64, _i64, _p],
    "nmb_adamw_step_hyper": [
        _p, _p, _p, _i32, _i64, _p, _p, _p, _i32, _i32, _p, _f32, _p, _p, _sz, _p,
    ],
}
_RESTYPES = {"nmb_last_error": ctypes.c_char_p}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load libnmb.so (once) and declare its signatures; raises if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m nano_megatron_amd.build` "
                    "(nano_megatron_amd has no CPU fallback)"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            lib.nmb_abi_version.restype = ctypes.c_int
            if lib.nmb_abi_version() != ABI_VERSION:
                raise RuntimeError(
                    f"{LIB_PATH} has ABI version {lib.nmb_abi_version()}, these bindings expect "
                    f"{ABI_VERSION}; rebuild it with `python -m nano_megatron_amd.build`"
                )
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    """Map a C status to the reference's exception types."""
    if status == NMB_OK:
        return
    message = load().nmb_last_error().decode(errors="replace")
    if status in (NMB_EINVAL, NMB_EUNSUPPORTED):
        raise ValueError(f"{what}: {message}")
    raise RuntimeError(f"{what}: {message}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return NMB_BF16
    if dtype == torch.float32:
        return NMB_F32
    raise ValueError(f"nano_megatron_amd kernels support float32 and bfloat16, got {dtype}; supported "
                     "precisions: params=compute=float32, or params=compute=bfloat16 with the fp32-master "
                     "optimizer")


def stream_of(t: torch.Tensor) -> int:
    """Handle of torch's current HIP stream on the tensor's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def i64x3(values) -> ctypes.Array:
    a, b, c = (int(v) for v in values)
    return (ctypes.c_int64 * 3)(a, b, c)


def ptr_array(values) -> ctypes.c_void_p:
    """A host ``void*[]`` passed as ``const void* const*`` (keeps the array alive)."""
    vals = [int(v) for v in values]
    arr = (ctypes.c_void_p * len(vals))(*vals)
    return ctypes.cast(arr, ctypes.c_void_p)


def i64_array(values) -> ctypes.Array:
    vals = [int(v) for v in values]
    return (ctypes.c_int64 * len(vals))(*vals)
