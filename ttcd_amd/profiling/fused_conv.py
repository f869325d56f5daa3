"""Drop-in for profiling/fused_conv.py (causal_dwconv_chunked, :51)."""
try:
    import ttcd_amd  # noqa: F401
except ImportError:  # only this directory is on sys.path
    import os
    import sys
    sys.path.append(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))

from ttcd_amd.conv import causal_dwconv_chunked  # noqa: E402,F401
