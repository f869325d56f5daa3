"""CPU oracle for the attention prologue (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this module, as
the checker.

  inv_freq_ref        fp32 1 / base ** (arange(0, dim, 2) / dim)
                      (fla/modules/rotary.py:418-425).
  tables_ref          cos/sin(fp32(t) * inv_freq) rounded to the dtype,
                      evaluated in float64 from the fp32 product
                      (fla/modules/rotary.py:441-490, pos_idx_in_fp32).
  rms_norm_ref        fla's RMSNorm forward (fla/modules/layernorm.py:219-251,
                      IS_RMS_NORM, HAS_WEIGHT): fp32 x, var = sum(x*x) / D,
                      rstd = 1 / sqrt(var + eps), y = (x * rstd) * w, rounded
                      to x's dtype.
  rope_ref            fla's rotary_embedding_kernel, non-interleaved
                      (fla/modules/rotary.py:93-107): o0 = x0*cos - x1*sin,
                      o1 = x0*sin + x1*cos in fp32, rounded to x's dtype.
  qk_norm_rope_ref    rms_norm_ref then rope_ref, on q and on k, as the
                      reference's four launches at profiling/patches.py:260-268.
  rotate_complex_f64  the same rotation as complex multiplication
                      (x0 + i x1) * exp(i theta) in float64 (textbook form).

Pins (tests/test_prologue.py): rope_ref == rotate_complex_f64 rounded to
fp32 and then to the dtype, bit for bit (each fp32 product of two 16-bit
values is exact, so the fp32 expression is the exact value rounded once),
and a planted sign / half swap fails that pin; position 0 is the identity;
<rope(q, m), rope(k, n)> depends only on m - n; norms are preserved;
rms_norm_ref within one rounding of a float64 evaluation, and closed forms
(constant rows, zero rows, power-of-two scale invariance); inv_freq_ref
against base ** (-2i / dim); tables_ref's column 0 (inv_freq 1) against
math.cos / math.sin of the position.
"""
from __future__ import annotations

import torch


def inv_freq_ref(dim: int, base: float) -> torch.Tensor:
    return 1.0 / (float(base) ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))


def tables_ref(inv_freq: torch.Tensor, rows: int, dtype=torch.bfloat16):
    """(cos, sin), each (rows, half): the fp32 product t * inv_freq, then
    cos / sin in float64 (correctly rounded to within 1 ulp), then dtype."""
    t = torch.arange(rows, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq.to(torch.float32))  # one fp32 rounding per product
    f64 = freqs.to(torch.float64)
    return torch.cos(f64).to(dtype), torch.sin(f64).to(dtype)


def rms_norm_ref(x: torch.Tensor, w: torch.Tensor | None, eps: float) -> torch.Tensor:
    xf = x.float()
    var = (xf * xf).sum(-1, keepdim=True) / x.shape[-1]
    rstd = 1.0 / torch.sqrt(var + eps)
    y = xf * rstd
    if w is not None:
        y = y * w.float()
    return y.to(x.dtype)


def rms_norm_f64(x: torch.Tensor, w: torch.Tensor | None, eps: float) -> torch.Tensor:
    """The same norm in float64 (unrounded), for pinning."""
    xd = x.double()
    y = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + eps)
    return y * w.double() if w is not None else y


def rope_ref(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
             seqlen_offset: int = 0) -> torch.Tensor:
    """x: (B, T, H, D); cos/sin: (TR, D/2) of x's dtype."""
    T, D = x.shape[1], x.shape[-1]
    R = D // 2
    c = cos[seqlen_offset:seqlen_offset + T].float()[None, :, None, :]
    s = sin[seqlen_offset:seqlen_offset + T].float()[None, :, None, :]
    xf = x.float()
    x0, x1 = xf[..., :R], xf[..., R:]
    o0 = x0 * c - x1 * s
    o1 = x0 * s + x1 * c
    return torch.cat([o0, o1], dim=-1).to(x.dtype)


def rotate_complex_f64(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                       seqlen_offset: int = 0) -> torch.Tensor:
    """(x0 + i x1) * (cos + i sin) in complex128 on the dtype-rounded tables,
    returned as float64 [real, imag] halves."""
    T, D = x.shape[1], x.shape[-1]
    R = D // 2
    xd = x.double()
    z = torch.complex(xd[..., :R], xd[..., R:])
    e = torch.complex(cos[seqlen_offset:seqlen_offset + T].double(),
                      sin[seqlen_offset:seqlen_offset + T].double())[None, :, None, :]
    r = z * e
    return torch.cat([r.real, r.imag], dim=-1)


def qk_norm_rope_ref(q, k, q_w, k_w, eps, cos, sin, seqlen_offset=0):
    if q_w is not None:
        q, k = rms_norm_ref(q, q_w, eps), rms_norm_ref(k, k_w, eps)
    return rope_ref(q, cos, sin, seqlen_offset), rope_ref(k, cos, sin, seqlen_offset)
