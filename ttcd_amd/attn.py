"""Dual-window attention entry points (host side of the HIP kernels).

Mirrors the reference's Python interface for this path:

* ``fused_dual_window_attn`` - profiling/fused_dual_attn.py:244-272
* ``lse_dual_window_attn`` / ``_fa3`` / ``_fa3_fast`` -
  profiling/lse_dual_attn.py:16-39, :74-99, :134-160

plus ``window_attn`` / ``band_attn`` (the single-window flash-attention call
those files make, ``flash_attn_func(q, k, v, causal=True,
window_size=(W-1, 0))``), ``lse_merge``, and the packed-sequence forms
``fused_dual_window_attn_varlen`` / ``band_attn_varlen`` (flash-attention's
varlen layout, the packed-batch path of fla/layers/attn.py:255-270 that the
reference's fused prefill declines).

Windows follow flash-attention's ``(W-1, 0)`` convention: key j is visible
to query i iff 0 <= i - j <= W - 1; a window of None or < 0 means full
causal. The softmax scale is head_dim ** -0.5, as in the reference. All
calls are forward-only, launch on torch's current stream, allocate only
their outputs and never synchronise.
"""
from __future__ import annotations

import torch

from . import _lib

_DT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16}

# Lazy online-softmax rescale threshold (log2 units) passed to the kernels:
# the reference row max moves only when a row's max exceeds it by more than
# 2^LAZY_RESCALE_LOG2. ``exact_max=True`` passes 0 instead: the exact running
# max of the reference kernel (profiling/fused_dual_attn.py:100-107), whose
# bf16 outputs it then reproduces bit for bit except where the dot-product
# order differs (98.6 % / 99.96 % of teacher / student outputs at config 1),
# for ~5 % more time.
LAZY_RESCALE_LOG2 = 8.0


def _rescale(exact_max: bool) -> float:
    return 0.0 if exact_max else LAZY_RESCALE_LOG2


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, fn: str):
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor) or t.dim() != 4:
            raise ValueError(f"{fn}: {name} must be a 4-D tensor (B, T, H, D)")
    if q.dtype not in _DT:
        raise ValueError(f"{fn}: dtype {q.dtype} not supported (bfloat16 or float16)")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"{fn}: q, k, v must share one dtype")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError(f"{fn}: q, k, v must be GPU (HIP) tensors")
    if not (q.device == k.device == v.device):
        raise ValueError(f"{fn}: q, k, v must be on one device")
    B, T, H, D = q.shape
    # Tk > Tq: a cached prefill, queries at the last Tq key positions
    if k.shape != v.shape or k.shape[0] != B or k.shape[1] < T or k.shape[3] != D:
        raise ValueError(f"{fn}: k/v must be (B, Tk, Hkv, D) with Tk >= Tq, matching q "
                         f"{tuple(q.shape)}, got {tuple(k.shape)} / {tuple(v.shape)}")
    HK = k.shape[2]
    if H % HK != 0:
        raise ValueError(f"{fn}: Hq ({H}) must be a multiple of Hkv ({HK})")
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        raise RuntimeError(f"{fn} is forward-only: autograd / gradient inputs are not supported; "
                           "call it under torch.no_grad() or torch.inference_mode()")
    return B, T, H, HK, D


def _ready(t: torch.Tensor) -> torch.Tensor:
    """t itself when the C ABI takes it as is (unit head_dim stride, element
    strides multiples of 8, 16-byte aligned base), else a contiguous copy: a
    q / k / v view of one fused projection output needs no copy."""
    if (t.stride(-1) == 1 and all(st % 8 == 0 for st in t.stride()[:-1])
            and t.data_ptr() % 16 == 0):
        return t
    return t.contiguous()


def _lse_ptr(t):
    return None if t is None else t.data_ptr()


def fused_dual_window_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           window_teacher: int, window_student: int, block_n: int = 64,
                           *, return_lse: bool = False, exact_max: bool = False):
    """Returns (o_teacher, o_student) of one pass over K/V.

    Same call as profiling/fused_dual_attn.py:244: q (B, T, H, D), k/v
    (B, T, HK, D) bf16/fp16, H % HK == 0; window_teacher None/-1 = full
    causal; window_student <= window_teacher (AssertionError otherwise).
    ``block_n`` is accepted for signature compatibility; the gfx950 kernel
    always sweeps 64-key tiles. Unlike the reference, window_student may be
    any value >= 1 and teacher == student windows of any alignment are exact.
    With ``return_lse=True`` also returns (lse_teacher, lse_student), fp32
    natural-log (B, H, T). ``exact_max=True`` keeps the reference kernel's
    exact running max (see LAZY_RESCALE_LOG2).

    k / v may be longer than q (Tk > Tq, a prefill onto a populated cache):
    the queries are then the last Tq positions, flash-attention's
    bottom-right aligned causal mask, which test/test_fused_dual_attn.py:
    275-293 asks of this call (a strict xfail for the reference kernel).
    """
    Tk = k.shape[1] if isinstance(k, torch.Tensor) and k.dim() == 4 else q.shape[1]
    if window_teacher is None or window_teacher < 0:
        window_teacher = Tk
    assert window_student <= window_teacher
    assert window_student >= 1, "window_student must be >= 1"
    if int(block_n) <= 0:
        raise ValueError("block_n must be positive")
    B, T, H, HK, D = _check_qkv(q, k, v, "fused_dual_window_attn")
    q, k, v = _ready(q), _ready(k), _ready(v)
    # o_t and o_s are the two contiguous halves of one allocation, so the
    # epilogue can run one o_proj GEMM over both without a copy
    both = torch.empty((2,) + tuple(q.shape), dtype=q.dtype, device=q.device)  # contiguous
    ot, os_ = both[0], both[1]
    lse_t = lse_s = None
    if return_lse:
        lse_t = torch.empty(B, H, T, device=q.device, dtype=torch.float32)
        lse_s = torch.empty(B, H, T, device=q.device, dtype=torch.float32)
    L = _lib.lib()
    _lib.check(L.ttcd_dual_window_attn_kv_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), ot.data_ptr(), os_.data_ptr(),
        _lse_ptr(lse_t), _lse_ptr(lse_s), B, T, k.shape[1], H, HK, D,
        _lib.strides4(q.stride()), _lib.strides4(k.stride()), _lib.strides4(v.stride()),
        _lib.strides4(ot.stride()), int(min(window_teacher, 2**31 - 1)),
        int(min(window_student, 2**31 - 1)), D ** -0.5, _rescale(exact_max), _DT[q.dtype],
        _stream(q.device)))
    if return_lse:
        return ot, os_, lse_t, lse_s
    return ot, os_


def band_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, band_lo: int, band_hi: int,
              *, return_lse: bool = False, exact_max: bool = False):
    """Causal attention over keys j with band_lo <= i - j < band_hi.

    (0, W) is flash_attn_func(q, k, v, causal=True, window_size=(W-1, 0));
    (WS, WT) is the far band of the LSE variant on unshifted tensors. Rows
    whose band is empty get o = 0 and lse = -inf.
    """
    B, T, H, HK, D = _check_qkv(q, k, v, "band_attn")
    Tk = k.shape[1]
    if band_hi is None or band_hi < 0:
        band_hi = max(Tk, band_lo + 1)
    if not (0 <= band_lo < band_hi):
        raise ValueError(f"band_attn: need 0 <= band_lo < band_hi, got ({band_lo}, {band_hi})")
    q, k, v = _ready(q), _ready(k), _ready(v)
    o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty(B, H, T, device=q.device, dtype=torch.float32) if return_lse else None
    L = _lib.lib()
    _lib.check(L.ttcd_band_attn_kv_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), _lse_ptr(lse),
        B, T, Tk, H, HK, D,
        _lib.strides4(q.stride()), _lib.strides4(k.stride()), _lib.strides4(v.stride()),
        _lib.strides4(o.stride()), int(min(band_lo, 2**31 - 1)), int(min(band_hi, 2**31 - 1)),
        D ** -0.5, _rescale(exact_max), _DT[q.dtype], _stream(q.device)))
    return (o, lse) if return_lse else o


def window_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int | None,
                *, return_lse: bool = False, exact_max: bool = False):
    """flash_attn_func(q, k, v, causal=True, window_size=(window-1, 0)) on gfx950;
    window None or < 0 = full causal. The "two separate calls" comparator.
    With k / v longer than q (a cached prefill), the queries are the last Tq
    positions (flash-attention's bottom-right alignment)."""
    T = k.shape[1] if isinstance(k, torch.Tensor) and k.dim() == 4 else q.shape[1]
    w = T if (window is None or window < 0) else window
    if w < 1:
        raise ValueError("window must be >= 1")
    return band_attn(q, k, v, 0, w, return_lse=return_lse, exact_max=exact_max)


def _check_varlen(q, k, v, cu_seqlens, max_seqlen, fn: str):
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor) or t.dim() != 3:
            raise ValueError(f"{fn}: {name} must be a 3-D packed tensor (total, H, D)")
    if q.dtype not in _DT:
        raise ValueError(f"{fn}: dtype {q.dtype} not supported (bfloat16 or float16)")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"{fn}: q, k, v must share one dtype")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError(f"{fn}: q, k, v must be GPU (HIP) tensors")
    total, H, D = q.shape
    if k.shape != v.shape or k.shape[0] != total or k.shape[2] != D:
        raise ValueError(f"{fn}: k/v must be (total, Hkv, D) matching q {tuple(q.shape)}, "
                         f"got {tuple(k.shape)} / {tuple(v.shape)}")
    HK = k.shape[1]
    if H % HK != 0:
        raise ValueError(f"{fn}: Hq ({H}) must be a multiple of Hkv ({HK})")
    if (not isinstance(cu_seqlens, torch.Tensor) or cu_seqlens.dim() != 1
            or cu_seqlens.dtype != torch.int32 or cu_seqlens.numel() < 2):
        raise ValueError(f"{fn}: cu_seqlens must be a 1-D int32 tensor of nseq + 1 offsets")
    if not (q.device == k.device == v.device == cu_seqlens.device):
        raise ValueError(f"{fn}: q, k, v and cu_seqlens must be on one device")
    if int(max_seqlen) < 1:
        raise ValueError(f"{fn}: max_seqlen must be >= 1")
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        raise RuntimeError(f"{fn} is forward-only: autograd / gradient inputs are not supported; "
                           "call it under torch.no_grad() or torch.inference_mode()")
    return total, H, HK, D, cu_seqlens.numel() - 1


def fused_dual_window_attn_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                  cu_seqlens: torch.Tensor, max_seqlen: int,
                                  window_teacher: int, window_student: int, *,
                                  return_lse: bool = False, exact_max: bool = False):
    """fused_dual_window_attn on packed sequences (flash-attention's varlen
    layout): q (total, H, D), k/v (total, HK, D); sequence b is rows
    cu_seqlens[b] .. cu_seqlens[b+1]-1 (int32 on the GPU, nseq + 1 entries)
    and attends causally within itself; max_seqlen bounds every length.
    Windows as fused_dual_window_attn. Returns (o_teacher, o_student) (and
    (lse_teacher, lse_student), fp32 (H, total), with ``return_lse``). Each
    sequence's outputs equal fused_dual_window_attn on that sequence alone.
    cu_seqlens is read on the GPU, so there is no host sync; the kernel
    clamps every sequence to the packed rows and max_seqlen, and rows
    outside every sequence are left unwritten."""
    if window_teacher is not None and window_teacher >= 0:
        assert window_student <= window_teacher
    assert window_student >= 1, "window_student must be >= 1"
    total, H, HK, D, nseq = _check_varlen(q, k, v, cu_seqlens, max_seqlen,
                                          "fused_dual_window_attn_varlen")
    wt = -1 if (window_teacher is None or window_teacher < 0) else window_teacher
    q, k, v = _ready(q), _ready(k), _ready(v)
    both = torch.empty((2,) + tuple(q.shape), dtype=q.dtype, device=q.device)
    ot, os_ = both[0], both[1]
    lse_t = lse_s = None
    if return_lse:
        lse_t = torch.empty(H, total, device=q.device, dtype=torch.float32)
        lse_s = torch.empty(H, total, device=q.device, dtype=torch.float32)
    if total == 0:  # every sequence empty: nothing to launch
        return (ot, os_, lse_t, lse_s) if return_lse else (ot, os_)
    L = _lib.lib()
    _lib.check(L.ttcd_dual_window_attn_varlen_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), ot.data_ptr(), os_.data_ptr(),
        _lse_ptr(lse_t), _lse_ptr(lse_s), cu_seqlens.data_ptr(), nseq, int(max_seqlen), total,
        H, HK, D, _lib.strides3(q.stride()), _lib.strides3(k.stride()),
        _lib.strides3(v.stride()), _lib.strides3(ot.stride()), int(min(wt, 2**31 - 1)),
        int(min(window_student, 2**31 - 1)), D ** -0.5, _rescale(exact_max), _DT[q.dtype],
        _stream(q.device)))
    if return_lse:
        return ot, os_, lse_t, lse_s
    return ot, os_


def band_attn_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     cu_seqlens: torch.Tensor, max_seqlen: int, band_lo: int, band_hi: int, *,
                     return_lse: bool = False, exact_max: bool = False):
    """band_attn on packed sequences (layout as fused_dual_window_attn_varlen);
    (0, W) is flash_attn_varlen_func(..., causal=True, window_size=(W-1, 0)).
    lse: fp32 (H, total)."""
    total, H, HK, D, nseq = _check_varlen(q, k, v, cu_seqlens, max_seqlen, "band_attn_varlen")
    if band_hi is None or band_hi < 0:
        band_hi = max(int(max_seqlen), band_lo + 1)
    if not (0 <= band_lo < band_hi):
        raise ValueError(f"band_attn_varlen: need 0 <= band_lo < band_hi, got ({band_lo}, "
                         f"{band_hi})")
    q, k, v = _ready(q), _ready(k), _ready(v)
    o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty(H, total, device=q.device, dtype=torch.float32) if return_lse else None
    if total == 0:  # every sequence empty: nothing to launch
        return (o, lse) if return_lse else o
    L = _lib.lib()
    _lib.check(L.ttcd_band_attn_varlen_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), _lse_ptr(lse),
        cu_seqlens.data_ptr(), nseq, int(max_seqlen), total, H, HK, D,
        _lib.strides3(q.stride()), _lib.strides3(k.stride()), _lib.strides3(v.stride()),
        _lib.strides3(o.stride()), int(min(band_lo, 2**31 - 1)), int(min(band_hi, 2**31 - 1)),
        D ** -0.5, _rescale(exact_max), _DT[q.dtype], _stream(q.device)))
    return (o, lse) if return_lse else o


def lse_merge(o_s: torch.Tensor, lse_s: torch.Tensor, o_f: torch.Tensor, lse_f: torch.Tensor,
              row_start: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """o_t = o_s*exp(lse_s-lt) + o_f*exp(lse_f-lt), lt = logaddexp(lse_s, lse_f), rows
    t >= row_start; rows below row_start copy o_s. o_*: (B, T, H, D), lse_*: (B, H, T) fp32.
    profiling/lse_dual_attn.py:106-131 and :151-159 (o_t[:, :WS] = o_s[:, :WS])."""
    B, T, H, D = o_s.shape
    if o_f.shape != o_s.shape or o_f.dtype != o_s.dtype or o_s.dtype not in _DT:
        raise ValueError("lse_merge: o_s and o_f must share shape and a bf16/fp16 dtype")
    if lse_s.shape != (B, H, T) or lse_f.shape != (B, H, T):
        raise ValueError("lse_merge: lse tensors must be (B, H, T)")
    o_s, o_f = o_s.contiguous(), o_f.contiguous()
    lse_s = lse_s.float().contiguous()
    lse_f = lse_f.float().contiguous()
    o_t = torch.empty_like(o_s) if out is None else out
    if o_t.shape != o_s.shape or o_t.stride() != o_s.stride():
        raise ValueError("lse_merge: out must be contiguous like o_s")
    L = _lib.lib()
    _lib.check(L.ttcd_lse_merge_fwd(
        o_s.data_ptr(), lse_s.data_ptr(), o_f.data_ptr(), lse_f.data_ptr(), o_t.data_ptr(),
        B, T, H, D, int(row_start), _lib.strides4(o_s.stride()), _DT[o_s.dtype],
        _stream(o_s.device)))
    return o_t


def lse_dual_window_attn(q, k, v, window_teacher: int, window_student: int, *,
                         exact_max: bool = False):
    """Student = window WS (with LSE); far band [WS, WT) (with LSE); teacher =
    exact LSE merge. profiling/lse_dual_attn.py:16-39 (flash-attn there, the
    gfx950 band kernel here). Requires WS < WT (AssertionError otherwise).
    One C call (ttcd_lse_dual_window_attn_fwd) with the far-band partial and
    both LSEs in a workspace allocated here; k / v may be longer than q (the
    queries are then the last Tq positions, as in fused_dual_window_attn)."""
    B, Tq, H, D = q.shape
    Tk = k.shape[1]
    WT = Tk if (window_teacher is None or window_teacher < 0) else window_teacher
    WS = window_student
    assert WS < WT
    if Tk <= WS:
        o_s = window_attn(q, k, v, WS, exact_max=exact_max)
        return o_s, o_s
    B, Tq, H, HK, D = _check_qkv(q, k, v, "lse_dual_window_attn")
    q, k, v = _ready(q), _ready(k), _ready(v)
    # o_t and o_s as the halves of one allocation (see fused_dual_window_attn)
    both = torch.empty((2,) + tuple(q.shape), dtype=q.dtype, device=q.device)
    ot, os_ = both[0], both[1]
    L = _lib.lib()
    WS_ = int(min(WS, 2**31 - 1))
    nbytes = L.ttcd_lse_dual_window_attn_workspace_bytes(B, Tq, Tk, H, D, WS_)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=q.device)
    _lib.check(L.ttcd_lse_dual_window_attn_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), ot.data_ptr(), os_.data_ptr(), B, Tq, Tk, H,
        HK, D, _lib.strides4(q.stride()), _lib.strides4(k.stride()), _lib.strides4(v.stride()),
        _lib.strides4(ot.stride()), int(min(WT, 2**31 - 1)), WS_, D ** -0.5,
        _rescale(exact_max), _DT[q.dtype], ws.data_ptr(), int(nbytes), _stream(q.device)))
    return ot, os_


def lse_dual_window_attn_fa3(q, k, v, window_teacher: int, window_student: int):
    """profiling/lse_dual_attn.py:74-99 (FA3 flavour). No FA3 on gfx950: the same band
    kernels serve it, and the far band needs no .contiguous() slice copies."""
    return lse_dual_window_attn(q, k, v, window_teacher, window_student)


def lse_dual_window_attn_fa3_fast(q, k, v, window_teacher: int, window_student: int):
    """profiling/lse_dual_attn.py:134-160 (two band calls + one-pass merge kernel);
    the student output is exactly the single-window call's output."""
    return lse_dual_window_attn(q, k, v, window_teacher, window_student)
