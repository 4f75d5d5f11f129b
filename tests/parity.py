"""Comparison bars of the parity tests, each scaled to the tensor it checks.

The north star's tolerances are rtol 1e-5 in fp32 and rtol 2e-2 / atol 1e-2 in
bf16.  An absolute atol says nothing about a gradient whose entries are all
below it (a zeroed gradient of magnitude 1e-3 passes atol 1e-2), so every bar
here reads atol relative to the largest magnitude of the expected tensor:

* ``assert_close_scaled`` (one kernel's output against the oracle's):
  ``|got - exp| <= rtol |exp| + atol max|exp|`` for every element, and the
  relative L2 error ``||got - exp|| / ||exp|| <= rtol``.  fp32: rtol = atol =
  1e-5; bf16: rtol 2e-2, atol 1e-2.  Where the expected tensor is exactly
  zero there is no magnitude to scale by, and atol bounds it absolutely.
* ``assert_bf16_grads`` (a whole bf16 model or block, where rounding builds up
  over the layers): the reference's own bf16 evaluation differs from the exact
  result (the fp32 evaluation of the same bf16 weights and inputs) by a
  relative L2 error ``e_ref`` that reaches 1.4% at 2 layers and 2.6% at the
  24-layer config-3 model (measured on the oracle), so two correct bf16
  implementations may differ from each other by about that much and a fixed
  2e-2 bar between them would reject a correct build.  The bar is instead
  ``e_got <= 1.5 e_ref + 5e-3`` per tensor, with both errors taken against the
  fp32 evaluation: this build is at most 1.5x as far from the exact gradient
  as the reference's own bf16 arithmetic is.  A zeroed gradient (e = 1) or one
  scaled by 1.05 (e >= 0.05 - e_ref) fails it whenever e_ref < 0.03, which
  ``assert_bf16_grads`` checks first, so the bar can never be wide enough to
  pass them (tests/test_parity_bars.py plants both).
* ``assert_loss_close``: bf16 losses within rtol 1e-3, fp32 within 1e-5.  A
  model with uniform logits has loss ln V, which the losses of these tests
  miss by 0.03-0.2 (9.07 against ln 8192 = 9.01 at config 1): rtol 2e-2 would
  let it pass, 1e-3 does not.

Set ``NMB_PARITY_LOG`` to a file path to append every comparison's figures as
JSON lines (the margins of a run, whether it passed or not).
"""

from __future__ import annotations

import json
import math
import os

import torch
from torch import Tensor

BF16_GRAD_FACTOR = 1.5
BF16_GRAD_FLOOR = 5e-3
BF16_GRAD_MAX_REF_ERR = 0.03


def _log(kind: str, name: str, **fields) -> None:
    path = os.environ.get("NMB_PARITY_LOG")
    if not path:
        return
    rec = {"kind": kind, "name": name, "test": os.environ.get("PYTEST_CURRENT_TEST", "")}
    rec.update({k: (float(v) if isinstance(v, (int, float)) else v) for k, v in fields.items()})
    with open(path, "a") as f:
        f.write(json.dumps(rec) + "\n")


def rel_l2(got: Tensor, exp: Tensor) -> float:
    got, exp = got.detach().double().cpu(), exp.detach().double().cpu()
    den = float(exp.norm())
    num = float((got - exp).norm())
    if den == 0.0:
        return 0.0 if num == 0.0 else math.inf
    return num / den


def bars(dtype: torch.dtype) -> tuple[float, float]:
    """(rtol, atol relative to max|exp|) for a tensor of ``dtype``."""
    return (1e-5, 1e-5) if dtype == torch.float32 else (2e-2, 1e-2)


def close_scaled(got: Tensor, exp: Tensor, rtol: float, atol: float) -> tuple[bool, float, float]:
    """(passes, worst element's error / its bound, relative L2 error)."""
    g, e = got.detach().double().cpu(), exp.detach().double().cpu()
    if g.shape != e.shape:
        raise AssertionError(f"shape {tuple(g.shape)} != {tuple(e.shape)}")
    if not torch.isfinite(g).all():
        return False, math.inf, math.inf
    diff = (g - e).abs()
    scale = float(e.abs().max())
    if scale == 0.0:
        # an all-zero expectation (a gradient that vanishes exactly, e.g. the
        # query gradient of a one-key softmax): no magnitude to scale by, so
        # the dtype's atol applies as an absolute bound and L2 is not formed
        worst = float(diff.max()) / atol
        return worst <= 1.0, worst, 0.0
    bound = rtol * e.abs() + atol * scale
    worst = float((diff / bound).max())
    l2 = rel_l2(g, e)
    return worst <= 1.0 and l2 <= rtol, worst, l2


def assert_close_scaled(got: Tensor, exp: Tensor, dtype: torch.dtype | None = None, *,
                        rtol: float | None = None, atol: float | None = None, msg: str = "") -> None:
    """Every element within ``rtol |exp| + atol max|exp|`` and the relative L2
    error within ``rtol``; the bars of ``dtype`` unless given."""
    dr, da = bars(dtype if dtype is not None else exp.dtype)
    rtol = dr if rtol is None else rtol
    atol = da if atol is None else atol
    ok, worst, l2 = close_scaled(got, exp, rtol, atol)
    _log("scaled", msg, worst=worst, rel_l2=l2, rtol=rtol, atol=atol)
    if not ok:
        raise AssertionError(f"{msg}: worst element at {worst:.3g} of its bound "
                             f"(rtol {rtol:g} + atol {atol:g} x max|exp|), relative L2 error {l2:.3g}")


def bf16_grad_error(got: Tensor, ref_bf16: Tensor, exact: Tensor) -> tuple[bool, float, float]:
    """(passes, this build's relative L2 error, the reference's), both against ``exact``."""
    if not torch.isfinite(got.detach().float()).all():
        return False, math.inf, rel_l2(ref_bf16, exact)
    e_got, e_ref = rel_l2(got, exact), rel_l2(ref_bf16, exact)
    return e_got <= BF16_GRAD_FACTOR * e_ref + BF16_GRAD_FLOOR, e_got, e_ref


def assert_bf16_grad(got: Tensor, ref_bf16: Tensor, exact: Tensor, msg: str = "") -> None:
    ok, e_got, e_ref = bf16_grad_error(got, ref_bf16, exact)
    direct = rel_l2(got, ref_bf16)
    _log("bf16_grad", msg, e_got=e_got, e_ref=e_ref, direct_rel_l2=direct)
    if e_ref >= BF16_GRAD_MAX_REF_ERR:
        raise AssertionError(f"{msg}: the reference's own bf16 error {e_ref:.3g} is too large for the "
                             f"bar to reject a gradient scaled by 1.05")
    if not ok:
        raise AssertionError(f"{msg}: relative L2 error {e_got:.3g} against the fp32 evaluation, "
                             f"above {BF16_GRAD_FACTOR} x the reference's {e_ref:.3g} + {BF16_GRAD_FLOOR}"
                             f" (direct difference from the bf16 oracle {direct:.3g})")


def assert_bf16_grads(ours, ref_bf16, ref_fp32) -> None:
    """Every parameter gradient of ``ours`` (a GPU module) against the bf16
    oracle and the fp32 oracle built from the same bf16 weights."""
    bf = dict(ref_bf16.named_parameters())
    fp = dict(ref_fp32.named_parameters())
    for name, p in ours.named_parameters():
        if p.grad is None:
            raise AssertionError(f"{name}: no gradient")
        assert_bf16_grad(p.grad, bf[name].grad, fp[name].grad, msg=name)


def assert_grads_scaled(ours, ref, dtype: torch.dtype) -> None:
    theirs = dict(ref.named_parameters())
    for name, p in ours.named_parameters():
        if p.grad is None:
            raise AssertionError(f"{name}: no gradient")
        assert_close_scaled(p.grad, theirs[name].grad, dtype, msg=name)


def loss_rtol(dtype: torch.dtype) -> float:
    return 1e-5 if dtype == torch.float32 else 1e-3


def assert_loss_close(got: Tensor | float, exp: Tensor | float, dtype: torch.dtype, msg: str = "loss") -> None:
    g = float(got.detach().float().cpu()) if isinstance(got, Tensor) else float(got)
    e = float(exp.detach().float().cpu()) if isinstance(exp, Tensor) else float(exp)
    rtol = loss_rtol(dtype)
    _log("loss", msg, got=g, exp=e, rel=abs(g - e) / max(abs(e), 1e-30), rtol=rtol)
    if not abs(g - e) <= rtol * abs(e):
        raise AssertionError(f"{msg}: {g!r} against {e!r}, relative difference {abs(g - e) / abs(e):.3g} "
                             f"above {rtol:g}")
