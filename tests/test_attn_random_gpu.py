"""Seeded random-shape parity sweep of the attention calls on the GPU.

Each case draws B, T, the head counts, D, the dtype, the windows and (for a
third of the cases) a cached prefill (Tq < Tk) from a fixed seed, so every run
checks the same cases. Windows cover w_S = 1, w_S = w_T, w_T >= T, full-causal
teachers, and unaligned values. Checks:
  * both outputs and both LSEs of fused_dual_window_attn against the fp32
    oracle (the tolerances of tests/test_attn_gpu.py, with the mean bounds
    scaled to the output's magnitude, see _assert_close; LSE within 1e-3);
  * the LSE-combination variant's teacher against the same oracle (w_S < w_T),
    allowing for its second rounding;
  * fused_dual_window_attn with exact_max=True against the oracle;
  * band_attn over random bands [lo, hi), rows with an empty band included
    (o = 0, lse = -inf), in both rescale modes.
"""
from __future__ import annotations

import random

import pytest
import torch

from conftest import random_cases
from oracle import attn_ref

pytestmark = pytest.mark.gpu

N_CASES = random_cases(400)


def _unit_roundoff(dtype):
    return 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11


def _assert_close(actual, expected, dtype, what, merged=False):
    """The reference test's bounds (tests/test_attn_gpu.py, from
    test_fused_dual_attn.py:88-110) plus the north-star bounds, with both mean
    bounds scaled to the output's magnitude. The absolute means (4e-4 bf16 /
    6e-5 f16 against the rounded oracle, 1e-3 against fp32) are sized for the
    reference's shapes, whose wide windows average outputs down to |o| ~ 0.05.
    Windows of a few keys here give |o| ~ 0.3-0.7, where one rounding of the
    output alone costs ~1e-3 against fp32, and a correct kernel's error against
    the rounded oracle is ~0.3 units of roundoff times |o|. So the rounded-oracle
    mean may reach max(absolute, 0.75 u mean|o|) (u = 2^-8 bf16, 2^-11 f16),
    and the fp32 mean may exceed the rounded oracle's own fp32 error by 1e-3.
    `merged` (the LSE variant's teacher, two roundings) doubles the first."""
    a = actual.float().cpu()
    e32 = expected.float().cpu()
    e = e32.to(dtype).float()
    diff = (a - e).abs()
    if dtype == torch.bfloat16:
        atol, rtol, mean_limit = 8e-3, 1e-2, 4e-4
    else:
        atol, rtol, mean_limit = 2e-3, 5e-3, 6e-5
    assert a.isfinite().all(), f"{what}: non-finite output"
    bad = diff > atol + rtol * e.abs()
    assert not bad.any(), (f"{what}: {bad.sum().item()} values exceed atol={atol}+rtol={rtol}; "
                           f"max err {diff.max().item():.3g}")
    limit = max(mean_limit, 0.75 * _unit_roundoff(dtype) * e.abs().mean().item())
    limit *= 2 if merged else 1
    assert diff.mean().item() <= limit, f"{what}: mean err {diff.mean().item():.3g} > {limit:.3g}"
    d32 = (a - e32).abs()
    assert d32.max().item() <= 2e-2, f"{what}: max err vs fp32 {d32.max().item():.3g}"
    own = (e - e32).abs().mean().item()
    assert d32.mean().item() <= 1e-3 + own, f"{what}: mean err vs fp32 {d32.mean().item():.3g}"


def _case(i):
    r = random.Random(1000 + i)
    D = r.choice([64, 128])
    HK = r.choice([1, 2, 3, 4])
    G = r.choice([1, 2, 3])
    B = r.choice([1, 1, 2])
    Tk = r.randint(1, 1500)
    Tq = Tk if r.random() < 0.67 else r.randint(1, Tk)
    dtype = r.choice([torch.bfloat16, torch.bfloat16, torch.float16])
    wt = r.choice([-1, Tk, Tk + r.randint(0, 300), r.randint(1, max(1, Tk)), r.randint(1, 600)])
    wt_eff = Tk if wt < 0 else wt
    ws = r.choice([1, wt_eff, r.randint(1, wt_eff), min(wt_eff, r.randint(1, 200))])
    return dict(B=B, Tq=Tq, Tk=Tk, H=HK * G, HK=HK, D=D, dtype=dtype, wt=wt, ws=ws, seed=i)


def _inputs(c):
    g = torch.Generator().manual_seed(7000 + c["seed"])
    q = torch.randn(c["B"], c["Tq"], c["H"], c["D"], generator=g).to(c["dtype"])
    k = torch.randn(c["B"], c["Tk"], c["HK"], c["D"], generator=g).to(c["dtype"])
    v = torch.randn(c["B"], c["Tk"], c["HK"], c["D"], generator=g).to(c["dtype"])
    return q, k, v


def _oracle(q, k, v, lo, hi):
    """Band [lo, hi) for the Tq queries at absolute positions Tk-Tq .. Tk-1."""
    B, Tq, H, D = q.shape
    Tk = k.shape[1]
    qp = torch.zeros(B, Tk, H, D, dtype=q.dtype)
    qp[:, Tk - Tq:] = q
    return attn_ref.band_reference(qp, k, v, lo, hi, rows=torch.arange(Tk - Tq, Tk),
                                   return_lse=True)


@pytest.mark.parametrize("i", range(N_CASES))
@torch.inference_mode()
def test_random_shape_matches_oracle(gpu, i):
    from ttcd_amd import fused_dual_window_attn, lse_dual_window_attn
    c = _case(i)
    print(f"case {i}: {c}", flush=True)
    q, k, v = _inputs(c)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    ot, os_, lt, ls = fused_dual_window_attn(qg, kg, vg, c["wt"], c["ws"], return_lse=True)
    xt, xs = fused_dual_window_attn(qg, kg, vg, c["wt"], c["ws"], exact_max=True)
    torch.cuda.synchronize()
    wt = c["Tk"] if c["wt"] < 0 else c["wt"]
    rt, rlt = _oracle(q, k, v, 0, wt)
    rs, rls = _oracle(q, k, v, 0, c["ws"])
    _assert_close(ot, rt, c["dtype"], f"case {i} teacher")
    _assert_close(os_, rs, c["dtype"], f"case {i} student")
    _assert_close(xt, rt, c["dtype"], f"case {i} teacher exact_max")
    _assert_close(xs, rs, c["dtype"], f"case {i} student exact_max")
    for got, want, what in ((lt, rlt, "lse_t"), (ls, rls, "lse_s")):
        g_, w_ = got.cpu(), want
        assert torch.equal(torch.isinf(g_), torch.isinf(w_)), f"case {i} {what}: -inf rows differ"
        fin = torch.isfinite(w_)
        if fin.any():
            assert (g_[fin] - w_[fin]).abs().max().item() < 1e-3, f"case {i} {what}"
    if c["ws"] < wt:
        lo_t, _ = lse_dual_window_attn(qg, kg, vg, c["wt"], c["ws"])
        torch.cuda.synchronize()
        _assert_close(lo_t, rt, c["dtype"], f"case {i} LSE-variant teacher", merged=True)



@pytest.mark.parametrize("i", range(random_cases(100)))
@torch.inference_mode()
def test_random_band_matches_oracle(gpu, i):
    """band_attn over a random band [lo, hi) (empty rows included: o = 0, lse = -inf),
    on the shapes of _case, both rescale modes, against the oracle."""
    from ttcd_amd import band_attn
    c = _case(5000 + i)
    r = random.Random(9000 + i)
    lo = r.choice([0, r.randint(0, 300), r.randint(0, c["Tk"])])
    hi = lo + r.choice([1, r.randint(1, 64), r.randint(1, c["Tk"] + 64)])
    print(f"case {i}: {c} band [{lo}, {hi})", flush=True)
    q, k, v = _inputs(c)
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    o, lse = band_attn(qg, kg, vg, lo, hi, return_lse=True)
    xo = band_attn(qg, kg, vg, lo, hi, exact_max=True)
    torch.cuda.synchronize()
    ro, rl = _oracle(q, k, v, lo, hi)
    empty = torch.isinf(rl)  # (B, H, Tq) rows with no key in the band
    assert torch.equal(torch.isinf(lse.cpu()), empty), f"case {i}: -inf rows differ"
    fin = ~empty
    if fin.any():
        assert (lse.cpu()[fin] - rl[fin]).abs().max().item() < 1e-3, f"case {i} lse"
    rows_empty = empty.permute(0, 2, 1)  # (B, Tq, H)
    assert (o.cpu()[rows_empty] == 0).all(), f"case {i}: empty rows not zero"
    _assert_close(o, ro, c["dtype"], f"case {i} band")
    _assert_close(xo, ro, c["dtype"], f"case {i} band exact_max")
