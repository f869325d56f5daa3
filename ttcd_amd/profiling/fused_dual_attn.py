"""Drop-in for profiling/fused_dual_attn.py (fused_dual_window_attn, :244)."""
try:
    import ttcd_amd  # noqa: F401
except ImportError:  # only this directory is on sys.path
    import os
    import sys
    sys.path.append(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))

from ttcd_amd.attn import fused_dual_window_attn  # noqa: E402,F401
