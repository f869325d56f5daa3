"""Seeded random-shape parity sweep of the attention calls on the GPU.

Each case draws B, T, the head counts, D, the dtype, the windows and (for a
third of the cases) a cached prefill (Tq < Tk) from a fixed seed, so every run
checks the same cases. Windows cover w_S = 1, w_S = w_T, w_T >= T, full-causal
teachers, and unaligned values. Checks:
  * both outputs and both LSEs of fused_dual_window_attn against the fp32
    oracle (the tolerances of tests/test_attn_gpu.py; LSE within 1e-3);
  * the LSE-combination variant's teacher against the same oracle (w_S < w_T),
    allowing for its second rounding;
  * fused_dual_window_attn with exact_max=True against the oracle.
"""
from __future__ import annotations

import random

import pytest
import torch

from oracle import attn_ref
from test_attn_gpu import _assert_close

pytestmark = pytest.mark.gpu

N_CASES = 120


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
        _assert_merged_close(lo_t, rt, c["dtype"], f"case {i} LSE-variant teacher")


def _assert_merged_close(actual, expected, dtype, what):
    """The LSE variant's teacher merges two outputs already rounded to the dtype
    (profiling/lse_dual_attn.py:32-38 merges flash-attention's rounded outputs
    the same way), so it carries two roundings: the pointwise bounds of
    _assert_close, twice its mean bound, and the north-star bounds vs fp32."""
    a = actual.float().cpu()
    e32 = expected.float().cpu()
    e = e32.to(dtype).float()
    atol, rtol, mean_limit = (8e-3, 1e-2, 4e-4) if dtype == torch.bfloat16 else (2e-3, 5e-3, 6e-5)
    diff = (a - e).abs()
    assert a.isfinite().all(), f"{what}: non-finite output"
    assert not (diff > atol + rtol * e.abs()).any(), f"{what}: max err {diff.max().item():.3g}"
    assert diff.mean().item() <= 2 * mean_limit, f"{what}: mean err {diff.mean().item():.3g}"
    d32 = (a - e32).abs()
    assert d32.max().item() <= 2e-2 and d32.mean().item() <= 1e-3, what
