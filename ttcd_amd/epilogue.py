"""Attention epilogue: one o_proj GEMM over the teacher and student attention
outputs, then their residual add + RMSNorm in one pass (host side of
epilogue.hip).

Replaces, in the patched TTT-layer forward (profiling/patches.py:289-298,
fuse_norm = True),

    teacher_attn_output = attn.o_proj(teacher_o)
    student_attn_output = attn.o_proj(student_o)
    student_output, _ = self.mlp_norm(student_attn_output, residual, True)
    hidden_states, residual = self.mlp_norm(teacher_attn_output, residual, True)

i.e. two GEMM launches and two fla RMSNorm launches (which read the residual
twice and also store the student's discarded residual sum), with one GEMM
(hipBLASLt, through torch) over the stacked outputs and one kernel.

    dual_residual_rmsnorm(attn_t, attn_s, residual, weight, eps)
        -> (hidden_states, residual_out, student_output)
    rmsnorm(x, weight, eps, residual=None)
        -> y, or (y, x + residual) with a residual (the model's other norms)
    add_rmsnorm(x, residual, weight, eps)
        -> (RMSNorm(h), h = residual + x rounded): a block's closing add + the
        next block's attn_norm
    fused_attn_epilogue(o_proj, mlp_norm, o_t, o_s, residual)
        drop-in for the call site above
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib

_DT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16,
       torch.float32: _lib.DTYPE_F32}


def dual_residual_rmsnorm(attn_t: torch.Tensor, attn_s: torch.Tensor, residual: torch.Tensor,
                          weight: torch.Tensor, eps: float):
    """For b in {t, s}: x_b = attn_b + residual (fp32), y_b = RMSNorm(x_b) * weight.
    Returns (y_t, x_t rounded to the dtype, y_s), as fla's
    ``rms_norm(attn_b, weight, residual=residual, prenorm=True)`` returns
    (y_b, x_b) (fla/modules/layernorm.py:715-764)."""
    for name, t in (("attn_t", attn_t), ("attn_s", attn_s), ("residual", residual),
                    ("weight", weight)):
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError(f"dual_residual_rmsnorm: {name} must be a tensor on a GPU (HIP) "
                             "device")
    if attn_t.shape != residual.shape or attn_s.shape != residual.shape:
        raise ValueError(f"dual_residual_rmsnorm: shapes differ: {tuple(attn_t.shape)}, "
                         f"{tuple(attn_s.shape)}, {tuple(residual.shape)}")
    # fla's own precondition (layernorm.py:738)
    assert residual.shape == attn_t.shape
    if (residual.dtype not in (torch.bfloat16, torch.float16)
            or attn_t.dtype != residual.dtype or attn_s.dtype != residual.dtype):
        raise ValueError("dual_residual_rmsnorm: activations must share bf16 or f16")
    H = residual.shape[-1]
    if weight.shape != (H,) or weight.dtype not in _DT:
        raise ValueError(f"dual_residual_rmsnorm: weight must be ({H},) of bf16, f16 or f32")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (attn_t, attn_s, residual, weight)):
        raise RuntimeError("dual_residual_rmsnorm is forward-only: autograd / gradient inputs "
                           "are not supported; call it under torch.no_grad()")
    a_t, a_s, res = attn_t.contiguous(), attn_s.contiguous(), residual.contiguous()
    w = weight.contiguous()
    # hidden_states and student_output are the two halves of one allocation, so
    # the TTT MLP can run its gate/up GEMM over both without a copy
    ys = torch.empty((2,) + tuple(res.shape), dtype=res.dtype, device=res.device)
    y_t, y_s = ys[0], ys[1]
    res_out = torch.empty_like(res)
    rows = res.numel() // H if H > 0 else 0
    if rows == 0:  # nothing to launch (an empty tensor's data pointer may be null)
        return y_t, res_out, y_s
    _lib.check(_lib.lib().ttcd_dual_residual_rmsnorm_fwd(
        a_t.data_ptr(), a_s.data_ptr(), res.data_ptr(), w.data_ptr(), _DT[w.dtype], float(eps),
        y_t.data_ptr(), res_out.data_ptr(), y_s.data_ptr(), rows, H, _DT[res.dtype],
        torch.cuda.current_stream(res.device).cuda_stream))
    return y_t, res_out, y_s


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            residual: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """fla's RMSNorm forward (fla/modules/layernorm.py:189-251, 715-764) on the
    GPU: ``RMSNorm(x) * weight`` rounded to x's dtype, or, with a residual, the
    prenorm form returning ``(RMSNorm(x + residual) * weight, x + residual)``
    with the variance of the unrounded fp32 sum. ``out`` (optional) receives y."""
    for name, t in (("x", x), ("weight", weight)) + ((("residual", residual),) if residual is not None else ()):
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError(f"rmsnorm: {name} must be a tensor on a GPU (HIP) device")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("rmsnorm: x must be bf16 or f16")
    H = x.shape[-1]
    if weight.shape != (H,) or weight.dtype not in _DT:
        raise ValueError(f"rmsnorm: weight must be ({H},) of bf16, f16 or f32")
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype):
        raise ValueError("rmsnorm: residual must match x in shape and dtype")
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x, residual, weight)):
        raise RuntimeError("rmsnorm is forward-only: call it under torch.no_grad()")
    x = x.contiguous()
    res = residual.contiguous() if residual is not None else None
    w = weight.contiguous()
    if out is None:
        y = torch.empty_like(x)
    else:
        if out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
            raise ValueError("rmsnorm: out must be contiguous and match x")
        y = out
    res_out = torch.empty_like(x) if res is not None else None
    rows = x.numel() // H if H > 0 else 0
    if rows > 0:
        _lib.check(_lib.lib().ttcd_rmsnorm_fwd(
            x.data_ptr(), res.data_ptr() if res is not None else None, w.data_ptr(),
            _DT[w.dtype], float(eps), y.data_ptr(),
            res_out.data_ptr() if res_out is not None else None, rows, H, _DT[x.dtype],
            torch.cuda.current_stream(x.device).cuda_stream))
    return y if res is None else (y, res_out)


def add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """``h = residual + x`` (a bf16/f16 torch add) followed by fla's plain
    RMSNorm of h, in one pass: returns (RMSNorm(h) * weight, h), with the norm
    taken on the ROUNDED h as the two separate launches take it
    (custom_models/ipttcd/modeling_ipttcdv9.py:870, then :627 of the next
    block)."""
    for name, t in (("x", x), ("residual", residual), ("weight", weight)):
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError(f"add_rmsnorm: {name} must be a tensor on a GPU (HIP) device")
    if x.dtype not in (torch.bfloat16, torch.float16) or residual.dtype != x.dtype \
            or residual.shape != x.shape:
        raise ValueError("add_rmsnorm: x and residual must match in shape and bf16/f16 dtype")
    H = x.shape[-1]
    if weight.shape != (H,) or weight.dtype not in _DT:
        raise ValueError(f"add_rmsnorm: weight must be ({H},) of bf16, f16 or f32")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (x, residual, weight)):
        raise RuntimeError("add_rmsnorm is forward-only: call it under torch.no_grad()")
    x, res, w = x.contiguous(), residual.contiguous(), weight.contiguous()
    y, h = torch.empty_like(x), torch.empty_like(x)
    rows = x.numel() // H if H > 0 else 0
    if rows > 0:
        _lib.check(_lib.lib().ttcd_add_rmsnorm_fwd(
            x.data_ptr(), res.data_ptr(), w.data_ptr(), _DT[w.dtype], float(eps), y.data_ptr(),
            h.data_ptr(), rows, H, _DT[x.dtype], torch.cuda.current_stream(x.device).cuda_stream))
    return y, h


def _stacked(o_t: torch.Tensor, o_s: torch.Tensor) -> torch.Tensor:
    """(2 * rows, cols) view of [o_t; o_s] when they are the two contiguous halves of
    one allocation (as fused_dual_window_attn returns them), else a stacked copy."""
    rows = o_t.numel() // o_t.shape[-1] if o_t.dim() >= 1 else 0
    n = o_t.numel()
    if (o_t.is_contiguous() and o_s.is_contiguous() and o_t.dtype == o_s.dtype
            and o_s.data_ptr() == o_t.data_ptr() + n * o_t.element_size()
            and o_t.untyped_storage().data_ptr() == o_s.untyped_storage().data_ptr()):
        return torch.as_strided(o_t, (2 * rows, o_t.shape[-1]), (o_t.shape[-1], 1))
    return torch.cat([o_t.reshape(rows, -1), o_s.reshape(rows, -1)], dim=0)


def fused_attn_epilogue(o_proj: torch.nn.Linear, mlp_norm, o_t: torch.Tensor,
                        o_s: torch.Tensor, residual: torch.Tensor):
    """Drop-in for profiling/patches.py:289-298 (fuse_norm = True): o_t, o_s are the
    teacher and student attention outputs (B, T, H, D) or (B, T, H*D); residual is
    (B, T, hidden). Returns (hidden_states, residual, student_output)."""
    B, T = residual.shape[0], residual.shape[1]
    o_t = o_t.reshape(B, T, -1)
    o_s = o_s.reshape(B, T, -1)
    if getattr(mlp_norm, "bias", None) is not None:
        raise NotImplementedError("fused_attn_epilogue: RMSNorm with bias")
    stacked = _stacked(o_t, o_s)
    proj = F.linear(stacked, o_proj.weight, o_proj.bias)  # hipBLASLt GEMM, one launch
    rows = B * T
    a_t = proj[:rows].view(B, T, -1)
    a_s = proj[rows:].view(B, T, -1)
    w = mlp_norm.weight
    if w is None:
        w = torch.ones(residual.shape[-1], dtype=torch.float32, device=residual.device)
    y_t, res_out, y_s = dual_residual_rmsnorm(a_t, a_s, residual, w, mlp_norm.eps)
    return y_t, res_out, y_s
