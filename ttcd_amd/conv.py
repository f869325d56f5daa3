"""Chunked causal depthwise conv (host side of the HIP kernel).

``causal_dwconv_chunked(x, conv)`` keeps the call of
profiling/fused_conv.py:51-61: x is the TTT MLP's (b, T, C, D) layout
(T chunks of C tokens, D channels), conv a depthwise
``nn.Conv1d(D, D, K, groups=D)``; the result equals
IPTTCDMLP._apply_ttt_conv with ttt_conv_causal=True
(custom_models/ipttcd/modeling_ipttcdv9.py:203-211) bit for bit:
fp32 accumulation over taps j = 0..K-1 in order, one RNE rounding. As in the
reference, conv.bias is not applied (the model builds these convs with
bias=False).
"""
from __future__ import annotations

import torch

from . import _lib

_DT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16,
       torch.float32: _lib.DTYPE_F32}


def causal_dwconv_x(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """y[n, c, d] = sum_j weight[d, j] * x[n, c-(K-1)+j, d] over the chunk axis
    c (zero left padding per chunk). x: (..., C, D), weight: (D, K)."""
    if not isinstance(x, torch.Tensor) or x.dim() < 2:
        raise ValueError("causal_dwconv: x must have at least 2 dims (..., C, D)")
    if x.dtype not in _DT or weight.dtype not in _DT:
        raise ValueError(f"causal_dwconv: unsupported dtypes {x.dtype}, {weight.dtype}")
    if not x.is_cuda or weight.device != x.device:
        raise ValueError("causal_dwconv: x and the conv weight must be on one GPU (HIP) device")
    C, D = x.shape[-2], x.shape[-1]
    if weight.dim() != 2 or weight.shape[0] != D:
        raise ValueError(f"causal_dwconv: weight must be (D={D}, K), got {tuple(weight.shape)}")
    if torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad):
        raise RuntimeError("causal_dwconv_chunked is forward-only: autograd / gradient inputs "
                           "are not supported; call it under torch.no_grad()")
    K = weight.shape[1]
    x = x.contiguous()
    w = weight.contiguous()
    y = torch.empty_like(x)
    N = x.numel() // max(1, C * D) if C * D > 0 else 0
    L = _lib.lib()
    _lib.check(L.ttcd_causal_dwconv_chunked_fwd(
        x.data_ptr(), w.data_ptr(), y.data_ptr(), N, C, D, K, _DT[x.dtype], _DT[w.dtype],
        torch.cuda.current_stream(x.device).cuda_stream))
    return y


def causal_dwconv_chunked(x: torch.Tensor, conv: torch.nn.Conv1d) -> torch.Tensor:
    """x: (b, T, C, D); conv: depthwise Conv1d(D, D, K, groups=D, padding=0).
    Equivalent to IPTTCDMLP._apply_ttt_conv with ttt_conv_causal=True."""
    b, T, C, D = x.shape
    K = conv.kernel_size[0]
    return causal_dwconv_x(x, conv.weight.view(D, K))
