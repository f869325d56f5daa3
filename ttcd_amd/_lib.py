"""ctypes binding of libttcd_amd.so (the C ABI declared in include/ttcd.h).

This is the whole "extension": torch tensors are unpacked into device
pointers, element strides and the current HIP stream handle, and passed to
the C entry points. There is no fallback path: if the library is missing or
fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
# TTCD_AMD_LIB overrides the library path (e.g. to A/B two builds of the kernels).
LIB_PATH = os.environ.get("TTCD_AMD_LIB") or os.path.join(_PKG_DIR, "lib", "libttcd_amd.so")

TTCD_OK = 0
TTCD_ERR_INVALID_ARGUMENT = 1
TTCD_ERR_UNSUPPORTED = 2
TTCD_ERR_HIP = 3

DTYPE_BF16 = 0
DTYPE_F16 = 1
DTYPE_F32 = 2

# Every extern "C" symbol of include/ttcd.h (checked by tests/test_abi.py).
EXPORTS = (
    "ttcd_status_string",
    "ttcd_last_error",
    "ttcd_abi_version",
    "ttcd_dual_window_attn_fwd",
    "ttcd_band_attn_fwd",
    "ttcd_dual_window_attn_kv_fwd",
    "ttcd_band_attn_kv_fwd",
    "ttcd_dual_window_attn_varlen_fwd",
    "ttcd_band_attn_varlen_fwd",
    "ttcd_lse_merge_fwd",
    "ttcd_lse_dual_window_attn_workspace_bytes",
    "ttcd_lse_dual_window_attn_fwd",
    "ttcd_lse_dual_window_attn_noalloc_scratch_bytes",
    "ttcd_lse_dual_window_attn_noalloc_fwd",
    "ttcd_causal_dwconv_chunked_fwd",
    "ttcd_qk_norm_rope_fwd",
    "ttcd_rope_table_fwd",
    "ttcd_dual_residual_rmsnorm_fwd",
    "ttcd_rmsnorm_fwd",
    "ttcd_add_rmsnorm_fwd",
    "ttcd_swiglu_fwd",
    "ttcd_ttt_features_fwd",
    "ttcd_ttt_proj_beta_t_fwd",
    "ttcd_ttt_scan_fwd",
    "ttcd_attn_schedule_coverage",
)

_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_fp = ctypes.c_void_p  # float* passed as a raw address
_i64x4 = ctypes.POINTER(ctypes.c_int64)
_i64x3 = ctypes.POINTER(ctypes.c_int64)

_SIGS = {
    "ttcd_status_string": (ctypes.c_char_p, [_i32]),
    "ttcd_last_error": (ctypes.c_char_p, []),
    "ttcd_abi_version": (_i32, []),
    "ttcd_dual_window_attn_fwd": (_i32, [
        _vp, _vp, _vp, _vp, _vp, _fp, _fp,
        _i32, _i32, _i32, _i32, _i32,
        _i64x4, _i64x4, _i64x4, _i64x4,
        _i32, _i32, ctypes.c_float, _i32, _vp]),
    "ttcd_band_attn_fwd": (_i32, [
        _vp, _vp, _vp, _vp, _fp,
        _i32, _i32, _i32, _i32, _i32,
        _i64x4, _i64x4, _i64x4, _i64x4,
        _i32, _i32, ctypes.c_float, _i32, _vp]),
    "ttcd_dual_window_attn_kv_fwd": (_i32, [
        _vp, _vp, _vp, _vp, _vp, _fp, _fp,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _i64x4, _i64x4, _i64x4, _i64x4,
        _i32, _i32, ctypes.c_float, ctypes.c_float, _i32, _vp]),
    "ttcd_band_attn_kv_fwd": (_i32, [
        _vp, _vp, _vp, _vp, _fp,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _i64x4, _i64x4, _i64x4, _i64x4,
        _i32, _i32, ctypes.c_float, ctypes.c_float, _i32, _vp]),
    "ttcd_dual_window_attn_varlen_fwd": (_i32, [
        _vp, _vp, _vp, _vp, _vp, _fp, _fp, _vp,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _i64x3, _i64x3, _i64x3, _i64x3,
        _i32, _i32, ctypes.c_float, ctypes.c_float, _i32, _vp]),
    "ttcd_band_attn_varlen_fwd": (_i32, [
        _vp, _vp, _vp, _vp, _fp, _vp,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _i64x3, _i64x3, _i64x3, _i64x3,
        _i32, _i32, ctypes.c_float, ctypes.c_float, _i32, _vp]),
    "ttcd_lse_merge_fwd": (_i32, [
        _vp, _fp, _vp, _fp, _vp,
        _i32, _i32, _i32, _i32, _i32, _i64x4, _i32, _vp]),
    "ttcd_lse_dual_window_attn_workspace_bytes": (ctypes.c_size_t, [
        _i32, _i32, _i32, _i32, _i32, _i32]),
    "ttcd_lse_dual_window_attn_fwd": (_i32, [
        _vp, _vp, _vp, _vp, _vp,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _i64x4, _i64x4, _i64x4, _i64x4,
        _i32, _i32, ctypes.c_float, ctypes.c_float, _i32, _vp, ctypes.c_size_t, _vp]),
    "ttcd_lse_dual_window_attn_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "ttcd_lse_dual_window_attn_noalloc_fwd": (_i32, [
        _vp, _vp, _vp, _vp, _vp,
        _i32, _i32, _i32, _i32, _i32, _i32,
        _i64x4, _i64x4, _i64x4, _i64x4,
        _i32, _i32, ctypes.c_float, ctypes.c_float, _i32, _vp]),
    "ttcd_causal_dwconv_chunked_fwd": (_i32, [
        _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _vp]),
    "ttcd_qk_norm_rope_fwd": (_i32, [
        _vp, _vp, _vp, _vp, _vp, _vp, _i32, ctypes.c_float,
        _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32,
        _i64x4, _i64x4, _i64x4, _i64x4, _i32, _i32, _vp]),
    "ttcd_rope_table_fwd": (_i32, [_vp, _vp, _fp, _i32, _i32, _i32, _vp]),
    "ttcd_dual_residual_rmsnorm_fwd": (_i32, [
        _vp, _vp, _vp, _vp, _i32, ctypes.c_float, _vp, _vp, _vp, _i64, _i32, _i32, _vp]),
    "ttcd_rmsnorm_fwd": (_i32, [
        _vp, _vp, _vp, _i32, ctypes.c_float, _vp, _vp, _i64, _i32, _i32, _vp]),
    "ttcd_add_rmsnorm_fwd": (_i32, [
        _vp, _vp, _vp, _i32, ctypes.c_float, _vp, _vp, _i64, _i32, _i32, _vp]),
    "ttcd_swiglu_fwd": (_i32, [_vp, _vp, _vp, _i64, _i32, _i64, _i64, _i64, _i32, _vp]),
    "ttcd_ttt_features_fwd": (_i32, [
        _vp, _vp, _i64, _vp, _vp, _i32, _i32, _vp, _vp, _vp,
        _i32, _i32, _i32, _i32, _i32, _vp]),
    "ttcd_ttt_proj_beta_t_fwd": (_i32, [
        _vp, _i64, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "ttcd_ttt_scan_fwd": (_i32, [
        _vp, _vp, ctypes.c_float, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "ttcd_attn_schedule_coverage": (_i32, [
        _i32, _i32, _i32, _i32, _i32, _vp, _vp]),
}

_lock = threading.Lock()
_lib = None


class TTCDError(RuntimeError):
    """A TTCD_ERR_* status returned by the C ABI."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def lib() -> ctypes.CDLL:
    """Load libttcd_amd.so once; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"ttcd_amd HIP library not built ({LIB_PATH} missing); run "
                    "`python -c 'import __graft_entry__ as g; g.build()'` or "
                    "`python -m ttcd_amd.build`")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def strides4(strides) -> ctypes.Array:
    return (ctypes.c_int64 * 4)(*[int(s) for s in strides])


def strides3(strides) -> ctypes.Array:
    return (ctypes.c_int64 * 3)(*[int(s) for s in strides])


def check(status: int) -> None:
    if status == TTCD_OK:
        return
    L = lib()
    msg = L.ttcd_last_error().decode(errors="replace")
    name = L.ttcd_status_string(status).decode()
    if status == TTCD_ERR_INVALID_ARGUMENT:
        raise ValueError(f"{name}: {msg}")
    raise TTCDError(status, f"{name}: {msg}")
