"""Attention epilogue (dual residual RMSNorm), CPU side: the oracle pinned by
float64 and closed forms, the C ABI's argument checks (before any HIP call),
and the Python layer's refusal of CPU tensors."""
from __future__ import annotations

import ctypes

import pytest
import torch

from oracle import attn_ref, epilogue_ref
from ttcd_amd import _lib, epilogue


def _rand(shape, dtype=torch.bfloat16, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def test_residual_out_is_the_rounded_sum():
    a, r = _rand((3, 50, 1024), seed=1), _rand((3, 50, 1024), seed=2, scale=4.0)
    _, res_out = epilogue_ref.residual_rms_norm_ref(a, r, None, 1e-6)
    want = (a.double() + r.double()).to(torch.bfloat16)
    rep = attn_ref.ulp_report(res_out, want)
    assert rep["max_ulp"] <= 1 and rep["bit_equal_pct"] > 99.9, rep


def test_norm_within_one_rounding_of_f64():
    a, r = _rand((2, 64, 960), seed=3), _rand((2, 64, 960), seed=4, scale=3.0)
    w = (1 + 0.1 * _rand((960,), torch.float32, seed=5)).to(torch.bfloat16)
    y, _ = epilogue_ref.residual_rms_norm_ref(a, r, w, 1e-6)
    y64, _ = epilogue_ref.residual_rms_norm_f64(a, r, w, 1e-6)
    rep = attn_ref.ulp_report(y, y64.float().to(torch.bfloat16))
    assert rep["max_ulp"] <= 1 and rep["bit_equal_pct"] > 99.0, rep


def test_closed_forms():
    H = 64
    w = torch.linspace(0.5, 1.5, H).to(torch.bfloat16)
    r = _rand((1, 3, H), seed=6)
    # a = -residual: zero sum, zero output
    y, res_out = epilogue_ref.residual_rms_norm_ref(-r, r, w, 1e-6)
    assert torch.all(y == 0) and torch.all(res_out == 0)
    # constant sum c: y = w * c / sqrt(c^2 + eps)
    a = torch.full((1, 1, H), 2.0).to(torch.bfloat16)
    r1 = torch.full((1, 1, H), 1.0).to(torch.bfloat16)
    y, _ = epilogue_ref.residual_rms_norm_ref(a, r1, w, 1e-6)
    want = (w.double() * 3.0 / (9.0 + 1e-6) ** 0.5).float().to(torch.bfloat16)
    assert torch.equal(y[0, 0], want)


def test_student_does_not_depend_on_teacher():
    r = _rand((1, 8, 256), seed=7)
    a_s = _rand((1, 8, 256), seed=8)
    w = torch.ones(256, dtype=torch.bfloat16)
    _, _, y1 = epilogue_ref.dual_residual_rms_norm_ref(_rand((1, 8, 256), seed=9), a_s, r, w, 1e-6)
    _, _, y2 = epilogue_ref.dual_residual_rms_norm_ref(_rand((1, 8, 256), seed=10), a_s, r, w, 1e-6)
    assert torch.equal(y1, y2)


_P = ctypes.c_void_p(0x10000)


def _call(**o):
    return _lib.lib().ttcd_dual_residual_rmsnorm_fwd(
        o.get("a", _P), _P, _P, o.get("w", _P), o.get("wdt", _lib.DTYPE_BF16), o.get("eps", 1e-6),
        o.get("y", _P), _P, _P, o.get("rows", 16), o.get("H", 1024),
        o.get("dtype", _lib.DTYPE_BF16), None)


@pytest.mark.parametrize("over,status", [
    (dict(a=None), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(w=None), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(rows=-1), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(H=0), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(H=1020), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(H=4096), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(dtype=_lib.DTYPE_F32), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(wdt=9), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(eps=-1e-6), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(a=ctypes.c_void_p(0x10002)), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(y=ctypes.c_void_p(0x10008)), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(w=ctypes.c_void_p(0x10004)), _lib.TTCD_ERR_UNSUPPORTED),
])
def test_rejects(over, status):
    assert _call(**over) == status
    assert _lib.lib().ttcd_last_error() != b""


def test_unaligned_fp32_weights_and_zero_rows_are_accepted_without_a_gpu():
    # zero rows: nothing to launch
    assert _call(rows=0, w=ctypes.c_void_p(0x10004), wdt=_lib.DTYPE_F32) == _lib.TTCD_OK


def test_python_layer_refuses_cpu_tensors():
    x = torch.zeros(2, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        epilogue.dual_residual_rmsnorm(x, x, x, torch.ones(64), 1e-6)
