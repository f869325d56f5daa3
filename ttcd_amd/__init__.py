"""ttcd_amd - MI355X (gfx950) native dual-window attention and chunked causal
depthwise conv for TTCD prefill.

Public API (reference signatures kept, see ttcd_amd/profiling for the
bare-module drop-in used by patches.py):

    fused_dual_window_attn(q, k, v, window_teacher, window_student, block_n=64)
    lse_dual_window_attn[_fa3[_fast]](q, k, v, window_teacher, window_student)
    causal_dwconv_chunked(x, conv)
    window_attn / band_attn / lse_merge
    fused_dual_window_attn_varlen / band_attn_varlen (packed sequences,
    flash-attention's varlen layout)
    qk_norm_rope / fused_qk_norm_rope / rope_tables / rope_inv_freq (attention
    prologue: q/k RMSNorm + rotary embedding in one pass)
    dual_residual_rmsnorm / fused_attn_epilogue (attention epilogue: one o_proj
    GEMM over both outputs, then both residual RMSNorms in one pass); rmsnorm
    swiglu / swiglu_mlp / ttt_features / ttt_mlp (the MLPs, ttcd_amd.ttt)
    IPTTCDv9Prefill / IPTTCDv9Cache / init_weights (the ipttcdv9 prefill end
    to end, optionally in chunks over a K/V cache, ttcd_amd.ipttcdv9)
"""
from .attn import (band_attn, band_attn_varlen, fused_dual_window_attn,
                   fused_dual_window_attn_varlen, lse_dual_window_attn,
                   lse_dual_window_attn_fa3, lse_dual_window_attn_fa3_fast, lse_merge,
                   window_attn)
from .conv import causal_dwconv_chunked, causal_dwconv_x
from .epilogue import dual_residual_rmsnorm, fused_attn_epilogue, rmsnorm
from .ipttcdv9 import IPTTCDv9Cache, IPTTCDv9Prefill, init_weights
from .prologue import fused_qk_norm_rope, qk_norm_rope, rope_inv_freq, rope_tables
from .ttt import swiglu, swiglu_mlp, ttt_features, ttt_mlp

__all__ = [
    "band_attn", "band_attn_varlen", "fused_dual_window_attn_varlen", "causal_dwconv_chunked", "causal_dwconv_x", "fused_dual_window_attn",
    "lse_dual_window_attn", "lse_dual_window_attn_fa3", "lse_dual_window_attn_fa3_fast",
    "lse_merge", "window_attn", "fused_qk_norm_rope", "qk_norm_rope", "rope_inv_freq",
    "rope_tables", "dual_residual_rmsnorm", "fused_attn_epilogue", "rmsnorm", "swiglu",
    "swiglu_mlp", "ttt_features", "ttt_mlp", "IPTTCDv9Prefill", "IPTTCDv9Cache",
    "init_weights",
]
