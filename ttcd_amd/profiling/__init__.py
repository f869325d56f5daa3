"""Bare-module drop-in directory.

The reference's profiling/patches.py imports the hot path by bare module name
from a directory on sys.path (``from fused_dual_attn import
fused_dual_window_attn``, ``from lse_dual_attn import
lse_dual_window_attn_fa3_fast``, ``from fused_conv import
causal_dwconv_chunked``; patches.py:227, :229, :414). Putting this directory
first on sys.path makes those imports resolve to the gfx950 kernels.
"""
