"""Attention prologue (q/k RMSNorm + rotary), CPU side: the oracle pinned by
closed forms and textbook identities, the C ABI's argument checks (they run
before any HIP call), and the Python layer's refusal of CPU tensors."""
from __future__ import annotations

import ctypes
import math

import pytest
import torch

from oracle import attn_ref, prologue_ref
from ttcd_amd import _lib, prologue, work


def _rand(shape, dtype=torch.bfloat16, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


# ---------------------------------------------------------------- oracle pins


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("offset", [0, 5, 4000])
def test_rope_ref_is_the_complex_rotation_rounded_once(D, offset):
    # fp32 products of two 16-bit values are exact, so the reference's fp32
    # expression equals the exact complex product rounded to fp32, then dtype.
    x = _rand((2, 37, 3, D), seed=1)
    cos, sin = prologue_ref.tables_ref(prologue_ref.inv_freq_ref(D, 1e6), offset + 37)
    got = prologue_ref.rope_ref(x, cos, sin, offset)
    want = prologue_ref.rotate_complex_f64(x, cos, sin, offset).float().to(torch.bfloat16)
    assert torch.equal(got, want)


def test_rope_ref_catches_a_sign_or_half_swap():
    # a plausible mistake (o1 = x0*s - x1*c) must fail the pin above
    x = _rand((1, 9, 2, 64), seed=2)
    cos, sin = prologue_ref.tables_ref(prologue_ref.inv_freq_ref(64, 1e4), 9)
    xf = x.float()
    c, s = cos.float()[None, :, None, :], sin.float()[None, :, None, :]
    wrong = torch.cat([xf[..., :32] * c - xf[..., 32:] * s, xf[..., :32] * s - xf[..., 32:] * c],
                      -1).to(x.dtype)
    assert not torch.equal(wrong, prologue_ref.rope_ref(x, cos, sin))


def test_position_zero_is_identity():
    x = _rand((1, 4, 5, 128), seed=3)
    cos, sin = prologue_ref.tables_ref(prologue_ref.inv_freq_ref(128, 1e6), 4)
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)
    assert torch.equal(prologue_ref.rope_ref(x, cos, sin)[:, 0], x[:, 0])


def test_relative_position_property():
    # <rope(q, m), rope(k, n)> depends only on m - n (fp32 inputs and tables)
    D = 64
    inv = prologue_ref.inv_freq_ref(D, 1e4).double()
    t = torch.arange(64, dtype=torch.float64)
    ang = torch.outer(t, inv)
    cos, sin = torch.cos(ang).float(), torch.sin(ang).float()
    q = _rand((1, 1, 1, D), torch.float32, seed=4).expand(1, 64, 1, D).contiguous()
    k = _rand((1, 1, 1, D), torch.float32, seed=5).expand(1, 64, 1, D).contiguous()
    rq = prologue_ref.rope_ref(q, cos, sin)[0, :, 0].double()
    rk = prologue_ref.rope_ref(k, cos, sin)[0, :, 0].double()
    for m, n, shift in ((10, 3, 20), (40, 40, 7), (5, 30, 25)):
        a = torch.dot(rq[m], rk[n])
        b = torch.dot(rq[m + shift], rk[n + shift])
        assert abs(float(a - b)) < 1e-4 * (1 + abs(float(a)))


def test_rotation_preserves_norms():
    x = _rand((2, 50, 3, 128), torch.float32, seed=6)
    cos, sin = prologue_ref.tables_ref(prologue_ref.inv_freq_ref(128, 1e6), 50, torch.float32)
    y = prologue_ref.rope_ref(x, cos, sin)
    assert torch.allclose(y.norm(dim=-1), x.norm(dim=-1), rtol=1e-5)


def test_rms_norm_ref_within_one_rounding_of_f64():
    x = _rand((4, 33, 3, 128), seed=7, scale=3.0)
    w = _rand((128,), seed=8, scale=0.2).float().add(1.0).to(torch.bfloat16)
    got = prologue_ref.rms_norm_ref(x, w, 1e-5)
    exact = prologue_ref.rms_norm_f64(x, w, 1e-5)
    rep = attn_ref.ulp_report(got, exact.float().to(torch.bfloat16))
    assert rep["max_ulp"] <= 1 and rep["bit_equal_pct"] > 99.0, rep


def test_rms_norm_closed_forms():
    D = 64
    w = torch.linspace(0.5, 1.5, D).to(torch.bfloat16)
    # constant row c: y = w * c / sqrt(c^2 + eps)
    for c in (3.0, -0.25, 17.0):
        x = torch.full((1, 1, 1, D), c).to(torch.bfloat16)
        want = (w.double() * c / math.sqrt(c * c + 1e-5)).float().to(torch.bfloat16)
        assert torch.equal(prologue_ref.rms_norm_ref(x, w, 1e-5)[0, 0, 0], want)
    # zero row stays zero
    z = torch.zeros(1, 1, 1, D, dtype=torch.bfloat16)
    assert torch.equal(prologue_ref.rms_norm_ref(z, w, 1e-5), z)
    # eps = 0: scaling by a power of two changes nothing
    x = _rand((2, 5, 2, D), seed=9)
    assert torch.equal(prologue_ref.rms_norm_ref(x, w, 0.0),
                       prologue_ref.rms_norm_ref((x.float() * 8).to(torch.bfloat16), w, 0.0))


def test_tables_and_inv_freq_closed_forms():
    D, base = 128, 1e6
    inv = prologue_ref.inv_freq_ref(D, base)
    want = torch.tensor([base ** (-2 * i / D) for i in range(D // 2)], dtype=torch.float64)
    assert torch.allclose(inv.double(), want, rtol=4e-7, atol=0)
    assert inv[0] == 1.0
    cos, sin = prologue_ref.tables_ref(inv, 70000)
    # column 0 has inv_freq 1: cos(t), sin(t) of the exact fp32 position
    for t in (0, 1, 2, 1000, 65535, 69999):
        assert cos[t, 0] == torch.tensor(math.cos(t)).to(torch.bfloat16)
        assert sin[t, 0] == torch.tensor(math.sin(t)).to(torch.bfloat16)


def test_prologue_bytes():
    # q and k read and written once + the table rows
    assert work.prologue_bytes(1, 65536, 16, 8, 128) == (
        2 * 65536 * 24 * 128 * 2 + 2 * 65536 * 64 * 2)


# ------------------------------------------------------------- C ABI checks

_P = ctypes.c_void_p(0x10000)


def _call(**over):
    lib = _lib.lib()
    B, T, Hq, Hkv, D = over.get("B", 1), over.get("T", 64), over.get("Hq", 4), \
        over.get("Hkv", 2), over.get("D", 128)
    qs = over.get("qs", _lib.strides4([T * Hq * D, Hq * D, D, 1]))
    ks = over.get("ks", _lib.strides4([T * Hkv * D, Hkv * D, D, 1]))
    return lib.ttcd_qk_norm_rope_fwd(
        over.get("q", _P), _P, over.get("qo", _P), _P, over.get("qw", _P), over.get("kw", _P),
        over.get("wdt", _lib.DTYPE_BF16), over.get("eps", 1e-5), over.get("cos", _P), _P,
        over.get("rows", 64), B, T, Hq, Hkv, D, qs, ks, qs, ks, over.get("off", 0),
        over.get("dtype", _lib.DTYPE_BF16), None)


@pytest.mark.parametrize("over,status", [
    (dict(q=None), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(cos=None), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(kw=None), _lib.TTCD_ERR_INVALID_ARGUMENT),            # one weight only
    (dict(T=0), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(D=96), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(dtype=_lib.DTYPE_F32), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(wdt=7), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(eps=-1.0), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(eps=float("nan")), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(off=-1), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(rows=63), _lib.TTCD_ERR_INVALID_ARGUMENT),           # T + offset > table rows
    (dict(off=1), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(qs=_lib.strides4([64 * 4 * 128, 4 * 128, 128, 2])), _lib.TTCD_ERR_INVALID_ARGUMENT),
    (dict(qs=_lib.strides4([64 * 4 * 128, 4 * 128, 132, 1])), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(q=ctypes.c_void_p(0x10008)), _lib.TTCD_ERR_UNSUPPORTED),
    (dict(qo=ctypes.c_void_p(0x10004)), _lib.TTCD_ERR_UNSUPPORTED),
])
def test_qk_norm_rope_rejects(over, status):
    assert _call(**over) == status
    assert _lib.lib().ttcd_last_error() != b""


def test_rope_table_rejects():
    lib = _lib.lib()
    inv = ctypes.c_void_p(0x20000)
    assert lib.ttcd_rope_table_fwd(None, _P, inv, 8, 64, _lib.DTYPE_BF16, None) == \
        _lib.TTCD_ERR_INVALID_ARGUMENT
    assert lib.ttcd_rope_table_fwd(_P, _P, None, 8, 64, _lib.DTYPE_BF16, None) == \
        _lib.TTCD_ERR_INVALID_ARGUMENT
    assert lib.ttcd_rope_table_fwd(_P, _P, inv, -1, 64, _lib.DTYPE_BF16, None) == \
        _lib.TTCD_ERR_INVALID_ARGUMENT
    assert lib.ttcd_rope_table_fwd(_P, _P, inv, 8, 0, _lib.DTYPE_BF16, None) == \
        _lib.TTCD_ERR_INVALID_ARGUMENT
    assert lib.ttcd_rope_table_fwd(_P, _P, inv, 8, 64, _lib.DTYPE_F32, None) == \
        _lib.TTCD_ERR_UNSUPPORTED
    # zero rows: nothing to do, no HIP call
    assert lib.ttcd_rope_table_fwd(_P, _P, inv, 0, 64, _lib.DTYPE_BF16, None) == _lib.TTCD_OK


def test_python_layer_refuses_cpu_tensors():
    q = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 4, 1, 64, dtype=torch.bfloat16)
    cos = torch.ones(4, 32, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        prologue.qk_norm_rope(q, k, None, None, 1e-5, cos, cos)
    with pytest.raises(ValueError, match="GPU"):
        prologue.rope_tables(torch.ones(32), 4)
