"""nmb_attn_bwd_noalloc through the C ABI against nmb_attn_bwd (caller
workspace): bit-identical dq / dK / dV on two calls in a row, the second with
a smaller problem, so the fixed scratch array is reused with stale contents
from the first call; and a problem beyond the array's size is rejected before
any launch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from nano_megatron_amd import _lib
from nano_megatron_amd import functional as Fn

pytestmark = pytest.mark.gpu


def _bwd(q, ks, vs, offs, o, do, lse, causal, q_offset, noalloc):
    dq = torch.empty_like(q)
    dks = [torch.empty_like(k) for k in ks]
    dvs = [torch.empty_like(v) for v in vs]
    b, sq, hq, d = q.shape
    _, sk, hkv, _ = ks[0].shape
    strides = lambda t: _lib.i64x3(Fn._eff_strides(t))  # noqa: E731
    args_head = (q.data_ptr(), _lib.ptr_array(k.data_ptr() for k in ks), _lib.ptr_array(v.data_ptr() for v in vs),
                 _lib.i64_array(offs), len(ks), o.data_ptr(), do.data_ptr(), lse.data_ptr(), dq.data_ptr(),
                 _lib.ptr_array(t.data_ptr() for t in dks), _lib.ptr_array(t.data_ptr() for t in dvs))
    args_tail = (b, hq, hkv, sq, sk, d, strides(q), strides(ks[0]), strides(o), 1 if causal else 0, q_offset, 0.0,
                 _lib.dtype_code(q.dtype), _lib.stream_of(q))
    if noalloc:
        _lib.call("nmb_attn_bwd_noalloc", *args_head, *args_tail)
    else:
        nbytes = ctypes.c_size_t(0)
        _lib.call("nmb_attn_bwd_workspace_bytes", b, hq, sq, ctypes.byref(nbytes))
        ws = torch.empty(max(nbytes.value, 16), dtype=torch.uint8, device=q.device)
        _lib.call("nmb_attn_bwd", *args_head, ws.data_ptr(), ws.numel(), *args_tail)
    return dq, dks, dvs


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_attn_bwd_noalloc_matches_workspace_entry(device, dtype) -> None:
    g = torch.Generator(device=device).manual_seed(2)
    # first call: config-3 attention (16 x 16 heads x 512); second: a smaller GQA
    # ring share with two blocks and a query offset
    cases = [(16, 16, 16, 512, 512, 64, 1, True, 0), (1, 4, 2, 200, 200, 64, 2, True, 200)]
    if dtype == torch.float32:
        cases = [(2, 4, 4, 256, 256, 64, 1, True, 0), (1, 2, 1, 100, 100, 64, 2, True, 100)]
    for b, hq, hkv, sq, sk, d, nb, causal, q_off in cases:
        q = torch.randn(b, sq, hq, d, device=device, generator=g).to(dtype)
        ks = [torch.randn(b, sk, hkv, d, device=device, generator=g).to(dtype) for _ in range(nb)]
        vs = [torch.randn(b, sk, hkv, d, device=device, generator=g).to(dtype) for _ in range(nb)]
        do = torch.randn(b, sq, hq, d, device=device, generator=g).to(dtype)
        offs = tuple(i * sk for i in range(nb))
        o, lse = Fn.attn_fwd_bshd(q, ks, vs, offs, causal=causal, q_offset=q_off, scale=None)
        ref = _bwd(q, ks, vs, offs, o, do, lse, causal, q_off, noalloc=False)
        got = _bwd(q, ks, vs, offs, o, do, lse, causal, q_off, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(got[0], ref[0])
        for a, r in zip(got[1] + got[2], ref[1] + ref[2]):
            assert torch.equal(a, r)


def test_attn_bwd_noalloc_rejects_oversized_problem(device) -> None:
    """batch x q_heads x seq_q above 1,048,576 is refused with EINVAL (nothing launched)."""
    fake = 256
    s = _lib.i64x3((0, 0, 0))
    ptrs = _lib.ptr_array([fake])
    with pytest.raises(ValueError, match="scratch"):
        _lib.call("nmb_attn_bwd_noalloc", fake, ptrs, ptrs, _lib.i64_array([0]), 1, fake, fake, fake, fake,
                  ptrs, ptrs, 4, 32, 8, 8193, 8193, 64, s, s, s, 1, 0, 0.0, _lib.NMB_BF16,
                  _lib.stream_of(torch.empty(1, device=device)))
