"""Attention prologue: per-head RMSNorm of q and k fused with the rotary
embedding (host side of prologue.hip).

Replaces, in the patched TTT-layer forward (profiling/patches.py:260-268;
the stock forward has the same steps at
custom_models/ipttcd/modeling_ipttcdv9.py:728-738),

    if attn.qk_norm:
        q, k = attn.q_norm(q), attn.k_norm(k)          # fla RMSNorm, twice
    if not attn.use_nope:
        q, k = attn.rotary(q, k, seqlen_offset=..., max_seqlen=...)

i.e. four launches that each read and write all of q or k, with one kernel
that reads and writes q and k once. Numerics follow fla's kernels
(fla/modules/layernorm.py:219-251, fla/modules/rotary.py:93-107): the norm's
output is rounded to the input dtype before the rotation, as between the
reference's two launches.

    rope_inv_freq(dim, base, device)            fla rotary.py:418-425
    rope_tables(inv_freq, rows, dtype)          fla rotary.py:441-490
    qk_norm_rope(q, k, q_w, k_w, eps, cos, sin, seqlen_offset=0)
    fused_qk_norm_rope(attn, q, k, seqlen_offset=0, max_seqlen=None)
        drop-in for the call site above on an fla ``Attention`` module
"""
from __future__ import annotations

import threading
import weakref

import torch

from . import _lib

_DT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16,
       torch.float32: _lib.DTYPE_F32}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def rope_inv_freq(dim: int, base: float, device=None) -> torch.Tensor:
    """1 / base ** (arange(0, dim, 2) / dim) in fp32, as
    RotaryEmbedding._compute_inv_freq (fla/modules/rotary.py:418-425, no YaRN)."""
    return 1.0 / (float(base) ** (torch.arange(0, dim, 2, device=device, dtype=torch.float32)
                                  / dim))


def rope_tables(inv_freq: torch.Tensor, rows: int,
                dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin), each (rows, len(inv_freq)) of `dtype`:
    cos(fp32(t) * inv_freq[i]) rounded to dtype, as
    RotaryEmbedding._update_cos_sin_cache with pos_idx_in_fp32
    (fla/modules/rotary.py:441-490). Computed on inv_freq's GPU."""
    if dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"rope_tables: dtype must be bf16 or f16, got {dtype}")
    if not isinstance(inv_freq, torch.Tensor) or not inv_freq.is_cuda or inv_freq.dim() != 1:
        raise ValueError("rope_tables: inv_freq must be a 1-D tensor on a GPU (HIP) device")
    inv = inv_freq.to(torch.float32).contiguous()
    half = inv.numel()
    cos = torch.empty(rows, half, dtype=dtype, device=inv.device)
    sin = torch.empty(rows, half, dtype=dtype, device=inv.device)
    _lib.check(_lib.lib().ttcd_rope_table_fwd(cos.data_ptr(), sin.data_ptr(), inv.data_ptr(),
                                              int(rows), half, _DT[dtype], _stream(inv)))
    return cos, sin


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_norm_weight: torch.Tensor | None,
                 k_norm_weight: torch.Tensor | None, eps: float, cos: torch.Tensor,
                 sin: torch.Tensor, seqlen_offset: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """q: (B, T, Hq, D), k: (B, T, Hkv, D) -> new contiguous (q, k) after
    per-head RMSNorm (skipped when both weights are None) and the
    non-interleaved rotary embedding at positions seqlen_offset .. + T - 1.
    cos, sin: (TR, D/2) tables of q's dtype."""
    for name, t in (("q", q), ("k", k), ("cos", cos), ("sin", sin)):
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError(f"qk_norm_rope: {name} must be a tensor on a GPU (HIP) device")
    if q.dim() != 4 or k.dim() != 4:
        raise ValueError(f"qk_norm_rope: q and k must be (B, T, H, D), got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}")
    B, T, Hq, D = q.shape
    if k.shape[0] != B or k.shape[1] != T or k.shape[3] != D:
        raise ValueError(f"qk_norm_rope: k {tuple(k.shape)} does not match q {tuple(q.shape)}")
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype:
        raise ValueError(f"qk_norm_rope: q and k must both be bf16 or f16, got {q.dtype}, "
                         f"{k.dtype}")
    # the reference's own preconditions (fla/modules/rotary.py:172-180)
    assert cos.dtype == sin.dtype, (
        f"cos and sin must have the same dtype, got {cos.dtype} and {sin.dtype}")
    assert q.dtype == cos.dtype, (
        f"Input and cos/sin must have the same dtype, got {q.dtype} and {cos.dtype}")
    assert D <= 256, "Only support D <= 256"
    if cos.dim() != 2 or cos.shape != sin.shape or cos.shape[1] * 2 != D:
        raise ValueError(f"qk_norm_rope: tables must be (TR, D/2 = {D // 2}), got "
                         f"{tuple(cos.shape)}, {tuple(sin.shape)}")
    assert seqlen_offset + T <= cos.shape[0], (
        f"seqlen_offset + T ({seqlen_offset + T}) exceeds the table rows ({cos.shape[0]})")
    if (q_norm_weight is None) != (k_norm_weight is None):
        raise ValueError("qk_norm_rope: give both norm weights or neither")
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (q, k, q_norm_weight, k_norm_weight)):
        raise RuntimeError("qk_norm_rope is forward-only: autograd / gradient inputs are not "
                           "supported; call it under torch.no_grad()")
    wq = wk = None
    w_code = _lib.DTYPE_F32
    if q_norm_weight is not None:
        if q_norm_weight.shape != (D,) or k_norm_weight.shape != (D,):
            raise ValueError(f"qk_norm_rope: norm weights must be ({D},)")
        if q_norm_weight.dtype not in _DT or k_norm_weight.dtype != q_norm_weight.dtype:
            raise ValueError("qk_norm_rope: norm weights must share one of bf16, f16, f32")
        wq, wk = q_norm_weight.contiguous(), k_norm_weight.contiguous()
        w_code = _DT[wq.dtype]
    q_out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    k_out = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    cos_c, sin_c = cos.contiguous(), sin.contiguous()
    _lib.check(_lib.lib().ttcd_qk_norm_rope_fwd(
        q.data_ptr(), k.data_ptr(), q_out.data_ptr(), k_out.data_ptr(),
        wq.data_ptr() if wq is not None else None, wk.data_ptr() if wk is not None else None,
        w_code, float(eps), cos_c.data_ptr(), sin_c.data_ptr(), cos_c.shape[0],
        B, T, Hq, k.shape[2], D, _lib.strides4(q.stride()), _lib.strides4(k.stride()),
        _lib.strides4(q_out.stride()), _lib.strides4(k_out.stride()), int(seqlen_offset),
        _DT[q.dtype], _stream(q)))
    return q_out, k_out


_tables_lock = threading.Lock()
# rotary module -> {(device, dtype): (cos, sin)}; like the module's own
# _cos_cached, a table is rebuilt only when more rows are needed
_tables: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()


def _cached_tables(rot, rows: int, dtype: torch.dtype):
    inv = rot.inv_freq
    key = (inv.device, dtype)
    with _tables_lock:
        per = _tables.get(rot)
        hit = per.get(key) if per is not None else None
    if hit is not None and hit[0].shape[0] >= rows:
        return hit
    tabs = rope_tables(inv, rows, dtype)
    with _tables_lock:
        _tables.setdefault(rot, {})[key] = tabs
    return tabs


def fused_qk_norm_rope(attn, q: torch.Tensor, k: torch.Tensor, seqlen_offset: int = 0,
                       max_seqlen: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Drop-in for profiling/patches.py:260-268 on an fla ``Attention`` module:
    applies ``attn.q_norm`` / ``attn.k_norm`` when ``attn.qk_norm`` and
    ``attn.rotary`` unless ``attn.use_nope``, in one kernel. The tables are
    built from the module's own ``rotary.inv_freq`` buffer for
    max(max_seqlen, T + seqlen_offset) positions, as the module's cache is."""
    T = q.shape[1]
    D = q.shape[-1]
    if getattr(attn, "qk_norm", False):
        qn, kn = attn.q_norm, attn.k_norm
        if getattr(qn, "bias", None) is not None or getattr(kn, "bias", None) is not None:
            raise NotImplementedError("fused_qk_norm_rope: RMSNorm with bias")
        if qn.eps != kn.eps:
            raise NotImplementedError("fused_qk_norm_rope: q_norm and k_norm eps differ")
        ones = None
        if qn.weight is None or kn.weight is None:
            ones = torch.ones(D, dtype=torch.float32, device=q.device)
        wq = qn.weight if qn.weight is not None else ones
        wk = kn.weight if kn.weight is not None else ones
        eps = float(qn.eps)
    else:
        wq = wk = None
        eps = 0.0
    rows = max(int(max_seqlen or 0), T + int(seqlen_offset))
    if getattr(attn, "use_nope", False):
        # identity rotation: cos = 1, sin = 0 reproduce the normed values exactly
        cos = torch.ones(rows, D // 2, dtype=q.dtype, device=q.device)
        sin = torch.zeros(rows, D // 2, dtype=q.dtype, device=q.device)
    else:
        rot = attn.rotary
        if getattr(rot, "interleaved", False):
            raise NotImplementedError("fused_qk_norm_rope: interleaved (GPT-J) rotary")
        if getattr(rot, "scale", None) is not None:
            raise NotImplementedError("fused_qk_norm_rope: XPos scaled rotary")
        if getattr(rot, "_yarn_attn_scaling", 1.0) != 1.0:
            raise NotImplementedError("fused_qk_norm_rope: YaRN mscale")
        cos, sin = _cached_tables(rot, rows, q.dtype)
    return qk_norm_rope(q, k, wq, wk, eps, cos, sin, seqlen_offset)
