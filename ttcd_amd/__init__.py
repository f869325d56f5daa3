"""ttcd_amd - MI355X (gfx950) native dual-window attention and chunked causal
depthwise conv for TTCD prefill.

Public API (reference signatures kept, see ttcd_amd/profiling for the
bare-module drop-in used by patches.py):

    fused_dual_window_attn(q, k, v, window_teacher, window_student, block_n=64)
    lse_dual_window_attn[_fa3[_fast]](q, k, v, window_teacher, window_student)
    causal_dwconv_chunked(x, conv)
    window_attn / band_attn / lse_merge
"""
from .attn import (band_attn, fused_dual_window_attn, lse_dual_window_attn,
                   lse_dual_window_attn_fa3, lse_dual_window_attn_fa3_fast, lse_merge,
                   window_attn)
from .conv import causal_dwconv_chunked, causal_dwconv_x

__all__ = [
    "band_attn", "causal_dwconv_chunked", "causal_dwconv_x", "fused_dual_window_attn",
    "lse_dual_window_attn", "lse_dual_window_attn_fa3", "lse_dual_window_attn_fa3_fast",
    "lse_merge", "window_attn",
]
