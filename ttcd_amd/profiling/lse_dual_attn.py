"""Drop-in for profiling/lse_dual_attn.py (lse_dual_window_attn :16,
lse_dual_window_attn_fa3 :74, lse_dual_window_attn_fa3_fast :134)."""
try:
    import ttcd_amd  # noqa: F401
except ImportError:  # only this directory is on sys.path
    import os
    import sys
    sys.path.append(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))

from ttcd_amd.attn import (lse_dual_window_attn, lse_dual_window_attn_fa3,  # noqa: E402,F401
                           lse_dual_window_attn_fa3_fast)
