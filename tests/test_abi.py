"""C ABI: the library loads, exports every function include/ttcd.h declares, and
rejects bad arguments with the documented status before touching the GPU."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from ttcd_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "ttcd.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ttcd_[a-z0-9_]+)\s*\(", text)))


def test_header_lists_match_binding():
    assert _declared() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.ttcd_abi_version() == 2


def test_status_strings():
    lib = _lib.lib()
    assert lib.ttcd_status_string(0) == b"TTCD_OK"
    assert lib.ttcd_status_string(1) == b"TTCD_ERR_INVALID_ARGUMENT"
    assert lib.ttcd_status_string(2) == b"TTCD_ERR_UNSUPPORTED"
    assert lib.ttcd_status_string(3) == b"TTCD_ERR_HIP"


def _attn_call(fn="dual", **over):
    """Call an attention entry point with fake (never dereferenced) 16-byte aligned
    pointers; argument checks run before any HIP call."""
    lib = _lib.lib()
    p = ctypes.c_void_p(0x10000)
    st = _lib.strides4([1 * 64 * 4 * 64, 4 * 64, 64, 1])
    args = dict(B=1, T=64, Hq=4, Hkv=2, D=64, wt=32, ws=16, scale=0.125, dtype=_lib.DTYPE_BF16,
                qs=st, ks=_lib.strides4([64 * 2 * 64, 2 * 64, 64, 1]), os=st, q=p, o=p)
    args.update(over)
    if fn == "dual":
        return lib.ttcd_dual_window_attn_fwd(
            args["q"], p, p, args["o"], p, None, None, args["B"], args["T"], args["Hq"],
            args["Hkv"], args["D"], args["qs"], args["ks"], args["ks"], args["os"], args["wt"],
            args["ws"], args["scale"], args["dtype"], None)
    return lib.ttcd_band_attn_fwd(
        args["q"], p, p, args["o"], None, args["B"], args["T"], args["Hq"], args["Hkv"],
        args["D"], args["qs"], args["ks"], args["ks"], args["os"], args.get("lo", 0),
        args.get("hi", 32), args["scale"], args["dtype"], None)


@pytest.mark.parametrize("over,status", [
    (dict(ws=33), _lib.TTCD_ERR_INVALID_ARGUMENT),          # ws > wt
    (dict(ws=0), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(Hq=3), _lib.TTCD_ERR_INVALID_ARGUMENT),           # Hq % Hkv
    (dict(D=96), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(dtype=_lib.DTYPE_F32), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(T=0), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(q=None), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(q=ctypes.c_void_p(0x10008)), _lib.TTCD_ERR_UNSUPPORTED),  # misaligned
    (dict(qs=_lib.strides4([64 * 4 * 64, 4 * 64, 64, 2])), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(qs=_lib.strides4([64 * 4 * 64, 4 * 64 + 4, 64, 1])), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(scale=0.0), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(ks=_lib.strides4([0, 2**25 + 8, 64, 1])), _lib.TTCD_ERR_UNSUPPORTED),  # 32-bit tile offsets
])
def test_dual_rejects(over, status):
    assert _attn_call("dual", **over) == status
    assert _lib.lib().ttcd_last_error()


@pytest.mark.parametrize("lo,hi", [(-1, 4), (5, 5), (7, 3)])
def test_band_rejects(lo, hi):
    assert _attn_call("band", lo=lo, hi=hi) == _lib.TTCD_ERR_INVALID_ARGUMENT


def test_conv_rejects():
    lib = _lib.lib()
    p = ctypes.c_void_p(0x10000)
    assert lib.ttcd_causal_dwconv_chunked_fwd(None, p, p, 1, 4, 8, 5, 0, 0, None) == 1
    assert lib.ttcd_causal_dwconv_chunked_fwd(p, p, p, 1, 4, 8, 0, 0, 0, None) == 1
    assert lib.ttcd_causal_dwconv_chunked_fwd(p, p, p, 1, 4, 8, 65, 0, 0, None) == 1
    assert lib.ttcd_causal_dwconv_chunked_fwd(p, p, p, 1, 4, 8, 5, 7, 0, None) == 1
    # empty tensors are a no-op (no launch)
    assert lib.ttcd_causal_dwconv_chunked_fwd(p, p, p, 0, 4, 8, 5, 0, 0, None) == 0


def test_merge_rejects():
    lib = _lib.lib()
    p = ctypes.c_void_p(0x10000)
    st = _lib.strides4([64 * 4 * 64, 4 * 64, 64, 1])
    assert lib.ttcd_lse_merge_fwd(p, p, p, p, None, 1, 64, 4, 64, 0, st, 0, None) == 1
    assert lib.ttcd_lse_merge_fwd(p, p, p, p, p, 1, 64, 4, 12, 0, st, 0, None) == 2
    assert lib.ttcd_lse_merge_fwd(p, p, p, p, p, 1, 64, 4, 64, -1, st, 0, None) == 1


def _varlen_call(fn="dual", **over):
    """Varlen entry points with fake (never dereferenced) 16-byte aligned pointers."""
    lib = _lib.lib()
    p = ctypes.c_void_p(0x10000)
    args = dict(cu=p, nseq=2, max_seqlen=64, total=100, Hq=4, Hkv=2, D=64, wt=32, ws=16,
                lo=0, hi=32, scale=0.125, rescale=8.0, dtype=_lib.DTYPE_BF16, q=p,
                qs=_lib.strides3([4 * 64, 64, 1]), ks=_lib.strides3([2 * 64, 64, 1]))
    args.update(over)
    common = (args["cu"], args["nseq"], args["max_seqlen"], args["total"], args["Hq"],
              args["Hkv"], args["D"], args["qs"], args["ks"], args["ks"], args["qs"])
    if fn == "dual":
        return lib.ttcd_dual_window_attn_varlen_fwd(
            args["q"], p, p, p, p, None, None, *common, args["wt"], args["ws"], args["scale"],
            args["rescale"], args["dtype"], None)
    return lib.ttcd_band_attn_varlen_fwd(
        args["q"], p, p, p, None, *common, args["lo"], args["hi"], args["scale"],
        args["rescale"], args["dtype"], None)


@pytest.mark.parametrize("over,status", [
    (dict(cu=None), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(nseq=0), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(max_seqlen=0), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(total=-1), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(ws=0), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(ws=33), _lib.TTCD_ERR_INVALID_ARGUMENT),           # ws > wt
    (dict(D=96), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(Hq=3), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(q=ctypes.c_void_p(0x10008)), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(qs=_lib.strides3([4 * 64, 64, 2])), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(scale=float("inf")), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(rescale=-1.0), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(rescale=17.0), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(rescale=float("nan")), _lib.TTCD_ERR_INVALID_ARGUMENT),
])
def test_dual_varlen_rejects(over, status):
    assert _varlen_call("dual", **over) == status
    assert _lib.lib().ttcd_last_error()


@pytest.mark.parametrize("lo,hi", [(-1, 4), (5, 5), (7, 3)])
def test_band_varlen_rejects(lo, hi):
    assert _varlen_call("band", lo=lo, hi=hi) == _lib.TTCD_ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("rescale", [-0.5, 16.5, float("inf"), float("nan")])
def test_kv_calls_reject_rescale_threshold(rescale):
    """rescale_log2 must lie in [0, 16] (0 = the reference kernel's exact running max)."""
    lib = _lib.lib()
    p = ctypes.c_void_p(0x10000)
    qs = _lib.strides4([64 * 4 * 64, 4 * 64, 64, 1])
    ks = _lib.strides4([64 * 2 * 64, 2 * 64, 64, 1])
    assert lib.ttcd_dual_window_attn_kv_fwd(
        p, p, p, p, p, None, None, 1, 64, 64, 4, 2, 64, qs, ks, ks, qs, 32, 16, 0.125, rescale,
        _lib.DTYPE_BF16, None) == _lib.TTCD_ERR_INVALID_ARGUMENT
    assert lib.ttcd_band_attn_kv_fwd(
        p, p, p, p, None, 1, 64, 64, 4, 2, 64, qs, ks, ks, qs, 0, 32, 0.125, rescale,
        _lib.DTYPE_BF16, None) == _lib.TTCD_ERR_INVALID_ARGUMENT
    assert b"rescale_log2" in lib.ttcd_last_error()


@pytest.mark.parametrize("rescale", [15.5, 16.0])
def test_f16_rescale_threshold_bounded_by_f16_range(rescale):
    """Under the lazy max a probability reaches 2^rescale_log2 and is rounded to
    the input dtype before PV; f16 rounds values >= 65520 to +inf, so F16 calls
    take at most 15 (bf16 keeps 16)."""
    lib = _lib.lib()
    p = ctypes.c_void_p(0x10000)
    qs = _lib.strides4([64 * 4 * 64, 4 * 64, 64, 1])
    ks = _lib.strides4([64 * 2 * 64, 2 * 64, 64, 1])
    assert lib.ttcd_dual_window_attn_kv_fwd(
        p, p, p, p, p, None, None, 1, 64, 64, 4, 2, 64, qs, ks, ks, qs, 32, 16, 0.125, rescale,
        _lib.DTYPE_F16, None) == _lib.TTCD_ERR_INVALID_ARGUMENT
    assert b"rescale_log2" in lib.ttcd_last_error()
    assert lib.ttcd_band_attn_kv_fwd(
        p, p, p, p, None, 1, 64, 64, 4, 2, 64, qs, ks, ks, qs, 0, 32, 0.125, rescale,
        _lib.DTYPE_F16, None) == _lib.TTCD_ERR_INVALID_ARGUMENT
    assert _varlen_call("dual", dtype=_lib.DTYPE_F16, rescale=rescale) == \
        _lib.TTCD_ERR_INVALID_ARGUMENT


def test_noalloc_lse_variant_rejects_rows_beyond_its_scratch():
    """The allocation-free LSE variant refuses, before any HIP call, a shape
    whose single query row does not fit its fixed scratch."""
    lib = _lib.lib()
    p = ctypes.c_void_p(0x10000)
    cap = lib.ttcd_lse_dual_window_attn_noalloc_scratch_bytes()
    assert cap == 64 << 20
    Hq = cap // (2 * 128 + 8) + 8            # one row of B * Hq * (2D + 8) bytes > cap
    qs = _lib.strides4([64 * Hq * 128, Hq * 128, 128, 1])
    ks = _lib.strides4([64 * 128, 128, 128, 1])
    st = lib.ttcd_lse_dual_window_attn_noalloc_fwd(
        p, p, p, p, p, 1, 64, 64, Hq, 1, 128, qs, ks, ks, qs, 32, 16, 128 ** -0.5, 8.0,
        _lib.DTYPE_BF16, None)
    assert st == _lib.TTCD_ERR_UNSUPPORTED
    assert b"scratch" in lib.ttcd_last_error()
    # the reference's strict gap (lse_dual_attn.py:20) holds here too
    assert lib.ttcd_lse_dual_window_attn_noalloc_fwd(
        p, p, p, p, p, 1, 64, 64, 4, 2, 64, _lib.strides4([64 * 256, 256, 64, 1]),
        _lib.strides4([64 * 128, 128, 64, 1]), _lib.strides4([64 * 128, 128, 64, 1]),
        _lib.strides4([64 * 256, 256, 64, 1]), 16, 16, 0.125, 8.0, _lib.DTYPE_BF16,
        None) == _lib.TTCD_ERR_INVALID_ARGUMENT


def test_ttt_scan_entry_points_reject_bad_arguments():
    lib = _lib.lib()
    p = ctypes.c_void_p(0x10000)
    # ttcd_ttt_proj_beta_t_fwd(pd, pd_stride, beta, beta_bs, pdt, B, nupd, chunk, H, dtype, stream)
    assert lib.ttcd_ttt_proj_beta_t_fwd(None, 64, p, 256, p, 1, 2, 128, 64, 0, None) == 1
    assert lib.ttcd_ttt_proj_beta_t_fwd(p, 32, p, 256, p, 1, 2, 128, 64, 0, None) == 1  # stride < H
    assert lib.ttcd_ttt_proj_beta_t_fwd(p, 64, p, 100, p, 1, 2, 128, 64, 0, None) == 1  # beta stride
    assert lib.ttcd_ttt_proj_beta_t_fwd(p, 64, p, 256, p, 1, 2, 128, 64, 2, None) == 2  # f32
    # ttcd_ttt_scan_fwd(dw, w_cur, lr, steps_t, w_next, nupd, nsteps, H, inter, dtype, stream)
    assert lib.ttcd_ttt_scan_fwd(p, p, 0.3, p, None, 2, 4, 64, 64, 0, None) == 1  # nsteps > nupd+1
    assert lib.ttcd_ttt_scan_fwd(None, p, 0.3, p, None, 2, 2, 64, 64, 0, None) == 1
    assert lib.ttcd_ttt_scan_fwd(p, p, 0.3, p, p, 0, 1, 64, 64, 0, None) == 1     # w_next, no update
    assert lib.ttcd_ttt_scan_fwd(p, p, float("nan"), p, None, 2, 2, 64, 64, 0, None) == 1
    assert lib.ttcd_ttt_scan_fwd(p, p, 0.3, p, None, 2, 2, 64, 64, 2, None) == 2
