"""CPU oracle for the attention epilogue (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker.

  residual_rms_norm_ref  fla's RMSNorm forward with a residual and prenorm
                         (fla/modules/layernorm.py:189-251 with HAS_RESIDUAL,
                         STORE_RESIDUAL_OUT, IS_RMS_NORM, HAS_WEIGHT;
                         LayerNormFunction.forward, :715-764): x = f32(a) +
                         f32(residual); residual_out = x rounded to the dtype;
                         var = sum(x*x) / H on the unrounded x;
                         y = (x * (1 / sqrt(var + eps))) * w rounded.
  dual_residual_rms_norm_ref
                         the teacher and the student call of
                         profiling/patches.py:296-298 on one residual.

Pins (tests/test_epilogue.py): residual_out == the float64 sum rounded to the
dtype; y within one rounding of a float64 evaluation; a = -residual gives
zeros; constant rows in closed form; the student output does not depend on
the teacher input.
"""
from __future__ import annotations

import torch


def residual_rms_norm_ref(a: torch.Tensor, residual: torch.Tensor, w: torch.Tensor | None,
                          eps: float):
    x = a.float() + residual.float()
    res_out = x.to(a.dtype)
    var = (x * x).sum(-1, keepdim=True) / a.shape[-1]
    rstd = 1.0 / torch.sqrt(var + eps)
    y = x * rstd
    if w is not None:
        y = y * w.float()
    return y.to(a.dtype), res_out


def residual_rms_norm_f64(a, residual, w, eps):
    x = a.double() + residual.double()
    y = x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps)
    return (y * w.double() if w is not None else y), x


def dual_residual_rms_norm_ref(a_t, a_s, residual, w, eps):
    y_t, res_out = residual_rms_norm_ref(a_t, residual, w, eps)
    y_s, _ = residual_rms_norm_ref(a_s, residual, w, eps)
    return y_t, res_out, y_s
