"""The C ABI (include/nmb.h) on the CPU: the library loads, exports every
declared symbol, and rejects bad arguments with a status and a message before
any device work (no kernel is launched by these tests)."""

from __future__ import annotations

import ctypes
import pathlib
import re

import pytest
import torch

from nano_megatron_amd import _lib

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "nmb.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:const\s+char\s*\*|int)\s+(nmb_\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_boundary() -> None:
    names = declared_functions()
    for expected in ("nmb_rmsnorm_fwd", "nmb_rmsnorm_bwd", "nmb_rope_apply", "nmb_swiglu_fwd",
                     "nmb_swiglu_bwd", "nmb_attn_fwd", "nmb_attn_bwd", "nmb_ce_fwd", "nmb_ce_bwd",
                     "nmb_last_error"):
        assert expected in names


def test_library_exports_every_declared_symbol() -> None:
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.nmb_abi_version() == 2


FAKE = 256  # a non-null, 16-byte aligned address that is never dereferenced


def test_rmsnorm_rejects_bad_arguments_without_launch() -> None:
    lib = _lib.load()
    st = lib.nmb_rmsnorm_fwd(FAKE, FAKE, FAKE, None, 4, 12, 1e-5, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EUNSUPPORTED
    assert b"multiple of 8" in lib.nmb_last_error()
    st = lib.nmb_rmsnorm_fwd(FAKE, FAKE, FAKE, None, 4, 64, 0.0, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL and b"eps" in lib.nmb_last_error()
    st = lib.nmb_rmsnorm_fwd(None, FAKE, FAKE, None, 4, 64, 1e-5, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL
    st = lib.nmb_rmsnorm_fwd(FAKE, FAKE, FAKE, None, 4, 64, 1e-5, 7, None)
    assert st == _lib.NMB_EUNSUPPORTED
    nbytes = ctypes.c_size_t(0)
    assert lib.nmb_rmsnorm_bwd_workspace_bytes(8192, 1024, ctypes.byref(nbytes)) == 0
    assert nbytes.value > 0 and nbytes.value % 4 == 0
    st = lib.nmb_rmsnorm_bwd(FAKE, FAKE, FAKE, None, FAKE, FAKE, FAKE, 4, 8192, 1024, 1e-5,
                             _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL and b"workspace" in lib.nmb_last_error()


def test_attention_rejects_bad_arguments_without_launch() -> None:
    lib = _lib.load()
    strides = _lib.i64x3((1024, 64, 64))
    ptrs = _lib.ptr_array([FAKE])
    offs = _lib.i64_array([0])
    st = lib.nmb_attn_fwd(FAKE, ptrs, ptrs, offs, 1, FAKE, FAKE, 1, 6, 4, 16, 16, 64,
                          strides, strides, strides, 1, 0, 0.0, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL
    assert b"must be divisible by KV heads" in lib.nmb_last_error()
    st = lib.nmb_attn_fwd(FAKE, ptrs, ptrs, offs, 1, FAKE, FAKE, 1, 4, 4, 16, 16, 96,
                          strides, strides, strides, 1, 0, 0.0, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EUNSUPPORTED and b"head_dim" in lib.nmb_last_error()
    st = lib.nmb_attn_fwd(FAKE, ptrs, ptrs, offs, 9, FAKE, FAKE, 1, 4, 4, 16, 16, 64,
                          strides, strides, strides, 1, 0, 0.0, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL and b"n_blocks" in lib.nmb_last_error()


def test_rope_and_swiglu_and_ce_reject_bad_arguments() -> None:
    lib = _lib.load()
    s = _lib.i64x3((0, 0, 0))
    st = lib.nmb_rope_apply(FAKE, FAKE, FAKE, FAKE, 16, None, 0, 0, 1, 4, 1, 7, s, s, 0,
                            _lib.NMB_F32, None)
    assert st == _lib.NMB_EINVAL and b"even" in lib.nmb_last_error()
    st = lib.nmb_rope_apply(FAKE, FAKE, FAKE, FAKE, 16, None, 0, 10, 1, 8, 1, 64,
                            _lib.i64x3((512, 64, 64)), _lib.i64x3((512, 64, 64)), 0,
                            _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL and b"exceed" in lib.nmb_last_error()
    st = lib.nmb_swiglu_fwd(FAKE, 10, FAKE, 10, FAKE, 10, 4, 10, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EUNSUPPORTED
    st = lib.nmb_ce_fwd(FAKE, 4, FAKE, 2, 8, -100, FAKE, FAKE, _lib.NMB_F32, None)
    assert st == _lib.NMB_EINVAL
    # fused gate/up + SwiGLU: F a multiple of 8, the [2F, K] weight under 2 GiB
    st = lib.nmb_gemm_bf16_swiglu(64, 12, 64, FAKE, 64, FAKE, 64, FAKE, 64, None, 0, None)
    assert st == _lib.NMB_EUNSUPPORTED and b"of 8" in lib.nmb_last_error()
    st = lib.nmb_gemm_bf16_swiglu(64, 1 << 20, 1024, FAKE, 1024, FAKE, 1024, FAKE, 1 << 20, None, 0,
                                  None)
    assert st == _lib.NMB_EUNSUPPORTED and b"2 GiB" in lib.nmb_last_error()
    st = lib.nmb_gemm_bf16_swiglu(64, 64, 64, FAKE, 64, FAKE, 64, FAKE, 32, None, 0, None)
    assert st == _lib.NMB_EINVAL and b"leading dimension" in lib.nmb_last_error()
    st = lib.nmb_gemm_bf16_swiglu(64, 64, 64, FAKE, 64, FAKE, 64, None, 0, FAKE, 64, None)
    assert st == _lib.NMB_EINVAL and b"2F" in lib.nmb_last_error()
    st = lib.nmb_gemm_bf16_swiglu(64, 64, 64, FAKE, 64, FAKE, 64, None, 0, None, 0, None)
    assert st == _lib.NMB_EINVAL and b"neither" in lib.nmb_last_error()


def test_gemm_f32out_rejects_bad_arguments() -> None:
    lib = _lib.load()
    st = lib.nmb_gemm_bf16_f32out(0, 0, 64, 64, 64, 1.0, FAKE, 64, FAKE, 64, 0.0, None, 64, None, 0,
                                  None)
    assert st == _lib.NMB_EINVAL and b"null" in lib.nmb_last_error()
    st = lib.nmb_gemm_bf16_f32out(0, 0, 64, 64, 64, 1.0, FAKE, 64, FAKE, 64, 0.0, FAKE, 62, None, 0,
                                  None)
    assert st == _lib.NMB_EINVAL and b"multiple of 4" in lib.nmb_last_error()
    st = lib.nmb_gemm_bf16_f32out(0, 0, 64, 64, 64, 1.0, FAKE, 64, FAKE, 64, 0.0, FAKE, 32, None, 0,
                                  None)
    assert st == _lib.NMB_EINVAL and b">= N" in lib.nmb_last_error()
    # a split plan needs its workspace
    st = lib.nmb_gemm_bf16_f32out(1, 1, 1024, 1024, 8192, 1.0, FAKE, 1024, FAKE, 1024, 0.0, FAKE,
                                  1024, None, 0, None)
    assert st == _lib.NMB_EINVAL and b"workspace" in lib.nmb_last_error()


def test_gemm_swiglu_bwd_rejects_bad_arguments() -> None:
    lib = _lib.load()
    st = lib.nmb_gemm_bf16_swiglu_bwd(1, 64, 64, 64, FAKE, 64, FAKE, 64, None, 128, FAKE, 128, None,
                                      0, None)
    assert st == _lib.NMB_EINVAL and b"null" in lib.nmb_last_error()
    st = lib.nmb_gemm_bf16_swiglu_bwd(2, 64, 64, 64, FAKE, 64, FAKE, 64, FAKE, 128, FAKE, 128, None,
                                      0, None)
    assert st == _lib.NMB_EINVAL and b"b_layout" in lib.nmb_last_error()
    st = lib.nmb_gemm_bf16_swiglu_bwd(1, 64, 12, 64, FAKE, 64, FAKE, 16, FAKE, 24, FAKE, 24, None,
                                      0, None)
    assert st == _lib.NMB_EUNSUPPORTED and b"multiples of 8" in lib.nmb_last_error()
    # gu narrower than [M, 2F]
    st = lib.nmb_gemm_bf16_swiglu_bwd(1, 64, 64, 64, FAKE, 64, FAKE, 64, FAKE, 64, FAKE, 128, None,
                                      0, None)
    assert st == _lib.NMB_EINVAL and b"[M, 2F]" in lib.nmb_last_error()
    st = lib.nmb_gemm_bf16_swiglu_bwd(1, 64, 64, 64, FAKE, 64, FAKE, 64, FAKE, 128, FAKE, 128, FAKE,
                                      32, None)
    assert st == _lib.NMB_EINVAL and b"act" in lib.nmb_last_error()


def test_gemm_f32_rejects_bad_arguments() -> None:
    lib = _lib.load()
    st = lib.nmb_gemm_f32(2, 0, 4, 4, 4, 1.0, FAKE, 4, FAKE, 4, 0.0, None, 4, FAKE, 4, None)
    assert st == _lib.NMB_EINVAL and b"a_layout" in lib.nmb_last_error()
    st = lib.nmb_gemm_f32(0, 0, 4, 4, 4, 1.0, FAKE, 3, FAKE, 4, 0.0, None, 4, FAKE, 4, None)
    assert st == _lib.NMB_EINVAL and b"leading dimension" in lib.nmb_last_error()
    st = lib.nmb_gemm_f32(0, 0, 4, 4, 4, 1.0, FAKE, 4, FAKE, 4, 1.0, None, 4, FAKE, 4, None)
    assert st == _lib.NMB_EINVAL and b"needs C" in lib.nmb_last_error()


def test_adamw_hyper_record_holds_the_double_formed_scalars() -> None:
    """nmb_adamw_hyper (host arithmetic only) writes the fp32 scalars of the
    update, each formed in double from the Python-float hyper-parameters and
    rounded once (data_parallel/_zero.py:176-189): checked against numpy."""
    import numpy as np

    lib = _lib.load()
    nb = ctypes.c_size_t(0)
    assert lib.nmb_adamw_hyper_bytes(ctypes.byref(nb)) == _lib.NMB_OK and nb.value == 36
    rec = (ctypes.c_uint8 * nb.value)()
    lr, b1, b2, eps, wd = 3e-4, 0.9, 0.95, 1e-8, 0.1
    for step in (1, 2, 7, 1000):
        assert lib.nmb_adamw_hyper(lr, b1, b2, eps, wd, step, rec) == _lib.NMB_OK
        got = np.frombuffer(bytes(rec), dtype=np.float32, count=8)
        has_decay = np.frombuffer(bytes(rec), dtype=np.int32, count=1, offset=32)[0]
        bc1, bc2 = 1.0 - b1**step, 1.0 - b2**step
        want = np.array([b1, 1.0 - b1, b2, 1.0 - b2, 1.0 - lr * wd, eps, bc2**0.5, -(lr / bc1)],
                        dtype=np.float64).astype(np.float32)
        assert np.array_equal(got, want), (step, got, want)
        assert has_decay == 1
    assert lib.nmb_adamw_hyper(lr, b1, b2, eps, 0.0, 1, rec) == _lib.NMB_OK
    assert np.frombuffer(bytes(rec), dtype=np.int32, count=1, offset=32)[0] == 0
    assert lib.nmb_adamw_hyper(lr, b1, b2, eps, wd, 0, rec) == _lib.NMB_EINVAL
    assert b"step" in lib.nmb_last_error()
    assert lib.nmb_adamw_hyper(lr, 1.0, b2, eps, wd, 1, rec) == _lib.NMB_EINVAL
    assert lib.nmb_adamw_hyper(lr, b1, b2, eps, wd, 1, None) == _lib.NMB_EINVAL
    st = lib.nmb_adamw_step_hyper(FAKE, FAKE, FAKE, 1, 16, FAKE, FAKE, FAKE, _lib.NMB_BF16,
                                  _lib.NMB_BF16, None, 1.0, None, FAKE, 1 << 20, None)
    assert st == _lib.NMB_EINVAL and b"hyper" in lib.nmb_last_error()


def test_python_wrapper_maps_status_to_exceptions() -> None:
    with pytest.raises(ValueError, match="multiple of 8"):
        _lib.call("nmb_rmsnorm_fwd", FAKE, FAKE, FAKE, None, 4, 12, 1e-5, _lib.NMB_BF16, None)
    with pytest.raises(ValueError):
        _lib.dtype_code(torch.float16)


def test_dropout_add_rejects_bad_arguments() -> None:
    lib = _lib.load()
    st = lib.nmb_dropout_add(FAKE, None, FAKE, 64, 1.0, 1, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL and b"[0, 1)" in lib.nmb_last_error()
    st = lib.nmb_dropout_add(FAKE, None, FAKE, 64, -0.5, 1, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL and b"[0, 1)" in lib.nmb_last_error()
    st = lib.nmb_dropout_add(None, None, FAKE, 64, 0.1, 1, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL and b"null" in lib.nmb_last_error()
    st = lib.nmb_dropout_add(FAKE, None, FAKE, -1, 0.1, 1, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL and b"negative" in lib.nmb_last_error()
    st = lib.nmb_dropout_add(FAKE, None, FAKE, 64, 0.1, 1, 7, None)
    assert st == _lib.NMB_EUNSUPPORTED and b"dtype" in lib.nmb_last_error()
    # nothing to do: no launch, OK
    assert lib.nmb_dropout_add(FAKE, None, FAKE, 0, 0.1, 1, _lib.NMB_BF16, None) == _lib.NMB_OK


def test_masked_attention_rejects_bad_dropout_and_mask_kind() -> None:
    lib = _lib.load()
    args = (FAKE, FAKE, FAKE, FAKE, FAKE, 1, 2, 2, 4, 4, 64, None, None, None)
    st = lib.nmb_attn_masked_fwd(*args, None, 0, None, 1, 0, 0.0, 1.0, 5, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL and b"dropout_p" in lib.nmb_last_error()
    st = lib.nmb_attn_masked_fwd(*args, None, 3, None, 1, 0, 0.0, 0.1, 5, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL and b"mask_kind" in lib.nmb_last_error()
    st = lib.nmb_attn_masked_fwd(*args, None, 1, None, 1, 0, 0.0, 0.1, 5, _lib.NMB_BF16, None)
    assert st == _lib.NMB_EINVAL and b"null mask" in lib.nmb_last_error()
