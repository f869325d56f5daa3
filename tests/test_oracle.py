"""Pins for the CPU oracle (the checker of every GPU parity test).

The reference ships no golden vectors for this path (its tests are seeded-random
and need flash_attn + CUDA), so the oracle is pinned by: a scalar float64
brute force with no shared code, closed forms, identities between independent
formulations, the reference's own CPU check (shifted-add vs nn.Conv1d,
test/test_fast_conv_patch.py:39-58), the committed fixtures in tests/golden/,
and planted mistakes (on the CPU, in a copy of the oracle's inputs) that must
fail the same checks.
"""
from __future__ import annotations

import math
import sys
import os

import numpy as np
import pytest
import torch

from oracle import attn_ref, conv_ref
from ttcd_amd import work

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _qkv(T, H, HK, D, seed, dtype=torch.bfloat16, B=1):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(B, T, h, D, generator=g).to(dtype) for h in (H, HK, HK))


# ----------------------------------------------------------------------------- counts
# the product's work counts (ttcd_amd/work.py), pinned by brute force
def test_band_pair_counts_brute_force():
    for T in (1, 7, 64, 129):
        i = np.arange(T)[:, None]
        j = np.arange(T)[None, :]
        d = i - j
        for lo, hi in ((0, 1), (0, 5), (3, 9), (0, T), (0, 10 * T), (2, T + 5)):
            want = int(((d >= lo) & (d < hi)).sum())
            assert work.band_pairs(T, lo, hi) == want
            if lo == 0:
                assert work.window_pairs(T, hi) == want


def test_headline_flop_constants():
    # Headline figures: P(65536, 8192) = 8192*8193/2 + (65536-8192)*8192 pairs per head,
    # and the teacher / student band FLOPs (4*D per pair, B=1, Hq=16, D=128).
    assert work.window_pairs(65536, 8192) == 503_320_576
    assert work.window_pairs(2048, 512) == 917_760
    assert abs(work.attn_flops(1, 16, 128, 65536, 8192) - 4.1232e12) < 1e8
    assert abs(work.attn_flops(1, 16, 128, 65536, 4096) - 2.1303e12) < 1e8


# ----------------------------------------------------------------------------- attention
@pytest.mark.parametrize("lo,hi", [(0, 1), (0, 4), (0, 13), (0, 100), (3, 7), (5, 6)])
def test_dense_matches_scalar_brute_force(lo, hi):
    q, k, v = _qkv(13, 4, 2, 8, seed=lo * 31 + hi, dtype=torch.float32, B=2)
    o, lse = attn_ref.dense_reference(q, k, v, hi, lo=lo, return_lse=True, dtype=torch.float64)
    bo, blse = attn_ref.brute_force_attention(q, k, v, lo, hi)
    assert torch.allclose(o, bo, atol=1e-12, rtol=0)
    assert torch.equal(torch.isinf(lse), torch.isinf(blse))
    fin = ~torch.isinf(blse)
    assert torch.allclose(lse[fin], blse[fin], atol=1e-12, rtol=0)


def test_brute_force_detects_off_by_one_window():
    """Planted mistake: a window one key too wide must be visible to the checks."""
    q, k, v = _qkv(20, 2, 1, 8, seed=3, dtype=torch.float32)
    o = attn_ref.dense_reference(q, k, v, 5, dtype=torch.float64)
    bad, _ = attn_ref.brute_force_attention(q, k, v, 0, 6)
    assert (o - bad).abs().max().item() > 2e-2


def test_closed_forms():
    q, k, v = _qkv(40, 4, 2, 16, seed=9, dtype=torch.float32)
    # window 1: each row attends only to itself
    o1 = attn_ref.dense_reference(q, k, v, 1)
    assert torch.allclose(o1, v.repeat_interleave(2, dim=2), atol=1e-6)
    # equal scores (q = 0): mean of v over the window, lse = log(count)
    z = torch.zeros_like(q)
    W = 7
    oz, lz = attn_ref.dense_reference(z, k, v, W, return_lse=True, dtype=torch.float64)
    vr = v.double().repeat_interleave(2, dim=2)
    for i in range(40):
        lo = max(0, i - W + 1)
        assert torch.allclose(oz[0, i], vr[0, lo:i + 1].mean(0), atol=1e-12)
        assert abs(lz[0, 0, i].item() - math.log(i - lo + 1)) < 1e-12
    # window >= T is plain causal attention
    assert torch.equal(attn_ref.dense_reference(q, k, v, 40), attn_ref.dense_reference(q, k, v, 500))
    assert torch.equal(attn_ref.dense_reference(q, k, v, -1), attn_ref.dense_reference(q, k, v, 40))


@pytest.mark.parametrize("lo,hi,rows", [(0, 37, None), (10, 50, None), (0, 200, [0, 5, 90, 91, 150]),
                                        (0, 17, list(range(100, 160)))])
def test_banded_matches_dense(lo, hi, rows):
    q, k, v = _qkv(160, 6, 3, 32, seed=hi)
    ro, rl = attn_ref.band_reference(q, k, v, lo, hi, rows=rows, chunk=48, return_lse=True,
                                     dtype=torch.float64)
    do, dl = attn_ref.dense_reference(q, k, v, hi, lo=lo, return_lse=True, dtype=torch.float64)
    idx = torch.arange(160) if rows is None else torch.tensor(rows)
    assert torch.allclose(ro, do[:, idx], atol=1e-12)
    assert torch.allclose(rl, dl[:, :, idx], atol=1e-12)


@pytest.mark.parametrize("lo,hi,qb", [(0, 37, 16), (10, 50, 7), (0, 200, 64), (0, 1, 33),
                                      (0, None, 50), (4, 5, 9)])
def test_blocked_matches_brute_force_and_banded(lo, hi, qb):
    """band_reference_blocked (the full-row checker of the 64K GPU tests) against the
    scalar float64 brute force and band_reference, over every row, with blocks that
    do not divide T and a GQA group of 3 (the head -> K/V head map is exercised)."""
    T = 130
    q, k, v = _qkv(T, 6, 2, 16, seed=(hi or T) + lo, dtype=torch.float32, B=2)
    ho = T if hi is None else hi
    bo, bl = attn_ref.brute_force_attention(q[:, :60], k[:, :60], v[:, :60], lo, ho)
    o, lse = attn_ref.band_reference_blocked(q, k, v, lo, hi, q_block=qb, return_lse=True)
    assert o.dtype == torch.float32 and o.shape == q.shape and lse.shape == (2, 6, T)
    assert torch.allclose(o[:, :60].double(), bo, atol=2e-6, rtol=0)
    fin = ~torch.isinf(bl)
    assert torch.equal(torch.isinf(lse[:, :, :60]), ~fin)
    assert torch.allclose(lse[:, :, :60].double()[fin], bl[fin], atol=2e-6, rtol=0)
    ro, rl = attn_ref.band_reference(q, k, v, lo, hi, return_lse=True)
    assert torch.allclose(o, ro, atol=2e-6, rtol=0)
    assert torch.allclose(lse[~torch.isinf(rl)], rl[~torch.isinf(rl)], atol=2e-6, rtol=0)


def test_blocked_detects_planted_head_map_mistake():
    """Planted mistake: K/V heads swapped in a copy of the inputs (the wrong GQA map)
    must move the blocked reference far from the brute force."""
    q, k, v = _qkv(40, 4, 2, 16, seed=5, dtype=torch.float32)
    o = attn_ref.band_reference_blocked(q, k.flip(2), v.flip(2), 0, 12, q_block=16)
    bo, _ = attn_ref.brute_force_attention(q, k, v, 0, 12)
    assert (o.double() - bo).abs().max().item() > 0.1


@pytest.mark.parametrize("ws,wt", [(16, 40), (1, 2), (30, 100)])
def test_lse_merge_identity(ws, wt):
    """softmax over disjoint bands [0, ws) + [ws, wt) merged by LSE == window wt
    (profiling/lse_dual_attn.py:6, the ring-attention identity)."""
    q, k, v = _qkv(90, 4, 2, 16, seed=ws, dtype=torch.float32)
    os_, ls = attn_ref.dense_reference(q, k, v, ws, return_lse=True, dtype=torch.float64)
    of, lf = attn_ref.dense_reference(q, k, v, wt, lo=ws, return_lse=True, dtype=torch.float64)
    ot, lt = attn_ref.dense_reference(q, k, v, wt, return_lse=True, dtype=torch.float64)
    mo, ml = attn_ref.lse_merge_reference(os_, ls, of, lf)
    assert torch.allclose(mo, ot, atol=1e-12)
    assert torch.allclose(ml, lt, atol=1e-12)


def test_reference_kernel_emulator_within_tolerance():
    """The emulated reference algorithm (64x64 blocks, segments A-E) agrees with the fp32
    masked softmax to the reference's own bf16 bounds; the narrow-gap segment too."""
    q, k, v = _qkv(300, 4, 2, 64, seed=73)
    for wt, ws in ((-1, 192), (256, 192), (300, 236)):
        et, es = attn_ref.emulate_reference_kernel(q, k, v, wt, ws)
        for W, o in ((wt, et), (ws, es)):
            mx, mean = attn_ref.error_stats(o, attn_ref.dense_reference(q, k, v, W))
            assert mx <= 2e-2 and mean <= 4e-4, (wt, ws, W, mx, mean)


def test_reference_kernel_emulator_sampled_blocks_equal_full_run():
    """Sampling (row_blocks, heads), as the headline numerics report does, gives the
    same bits as those blocks of the whole emulation."""
    q, k, v = _qkv(300, 4, 2, 64, seed=74)
    ft, fs = attn_ref.emulate_reference_kernel(q, k, v, 256, 128)
    st, ss = attn_ref.emulate_reference_kernel(q, k, v, 256, 128, row_blocks=[64, 256],
                                               heads=[1, 2])
    for r0, r1 in ((64, 128), (256, 300)):
        for h in (1, 2):
            assert torch.equal(st[:, r0:r1, h], ft[:, r0:r1, h])
            assert torch.equal(ss[:, r0:r1, h], fs[:, r0:r1, h])
    assert not st[:, :64].any() and not st[:, :, 0].any()


def test_ulp_report_known_values():
    one = torch.tensor([1.0], dtype=torch.bfloat16)
    nxt = torch.tensor([1.0078125], dtype=torch.bfloat16)  # 1 + 2^-7: next bf16 after 1
    assert attn_ref.ulp_report(one, nxt)["max_ulp"] == 1
    assert attn_ref.ulp_report(nxt, one)["bit_equal_pct"] == 0.0
    pz = torch.tensor([0.0], dtype=torch.bfloat16)
    nz = torch.tensor([-0.0], dtype=torch.bfloat16)
    assert attn_ref.ulp_report(pz, nz)["max_ulp"] == 0
    tiny = torch.tensor([1], dtype=torch.int16).view(torch.bfloat16)      # +min subnormal
    ntiny = torch.tensor([-32767], dtype=torch.int16).view(torch.bfloat16)  # -min subnormal
    assert attn_ref.ulp_report(tiny, ntiny)["max_ulp"] == 2


# ----------------------------------------------------------------------------- conv
def _conv_case(shape, K, xdt, wdt, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g).to(xdt)
    w = torch.randn(shape[-1], K, generator=g).to(wdt)
    return x, w


def _bits(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)


@pytest.mark.parametrize("xdt,wdt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                     (torch.bfloat16, torch.float16), (torch.float16, torch.bfloat16)])
@pytest.mark.parametrize("K", [1, 3, 5, 9])
def test_conv_c_equals_numpy(xdt, wdt, K):
    x, w = _conv_case((2, 3, 29, 24), K, xdt, wdt, seed=K)
    assert torch.equal(_bits(conv_ref.dwconv_c(x, w)), _bits(conv_ref.dwconv_numpy(x, w)))


@pytest.mark.parametrize("K", [1, 2, 5, 7])
def test_conv_taps_match_model_conv1d(K):
    """fp32 accumulation (no final rounding) vs the model's rearrange/pad/conv1d in fp64:
    within the sequential-summation bound, so every tap index and the zero padding are
    pinned; the final bf16 rounding is the oracle's RNE of that fp32 value."""
    x, w = _conv_case((2, 3, 31, 16), K, torch.bfloat16, torch.bfloat16, seed=K + 10)
    acc = conv_ref.dwconv_c(x.float(), w.float())          # fp32 out, products exact
    exact = conv_ref.conv1d_reference(x, w)
    absum = conv_ref.conv1d_reference(x.float().abs(), w.float().abs())
    assert ((acc.double() - exact).abs() <= K * 2.0 ** -24 * absum + 1e-30).all()
    assert torch.equal(_bits(conv_ref.dwconv_c(x, w)), _bits(conv_ref.round_c(acc, torch.bfloat16)))
    # planted mistake: taps in reverse order must violate the same bound
    bad = conv_ref.dwconv_c(x.float(), w.float().flip(1))
    if K > 1:
        assert not ((bad.double() - exact).abs() <= K * 2.0 ** -24 * absum + 1e-30).all()


def test_conv_shifted_add_matches_conv1d():
    """The reference's own CPU check (test/test_fast_conv_patch.py:39-58) restated."""
    torch.manual_seed(0)
    b, t, c, d, k = 2, 3, 17, 8, 5
    x = torch.randn(b, t, c, d)
    conv = torch.nn.Conv1d(d, d, kernel_size=k, padding=0, groups=d, bias=False)
    w = conv.weight.detach().view(d, k)
    y = x * w[:, k - 1]
    for i in range(1, k):
        y[:, :, i:, :] += x[:, :, :-i, :] * w[:, k - 1 - i]
    ref = conv_ref.conv1d_reference(x, w)
    assert (ref - y.double()).abs().max().item() < 1e-5
    assert (ref - conv_ref.dwconv_c(x, w).double()).abs().max().item() < 1e-5


def test_conv_identity_init():
    """Tap K-1 = 1 (modeling_ipttcdv9.py:977-994) reproduces x exactly."""
    x, _ = _conv_case((1, 2, 20, 16), 5, torch.bfloat16, torch.bfloat16, seed=1)
    w = torch.zeros(16, 5, dtype=torch.bfloat16)
    w[:, 4] = 1
    assert torch.equal(conv_ref.dwconv_c(x, w), x)


def test_rounding_encoders_match_torch():
    vals = [0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.0e-41, -2.5e-39, 65504.0, 65519.0,
            65520.0, 1e30, -1e-8, 5.960464477539063e-08, 2.9802322387695312e-08,
            8.940696716308594e-08, 6.103515625e-05, 6.097555160522461e-05, float("inf"),
            float("-inf")]
    g = torch.Generator().manual_seed(0)
    src = torch.cat([torch.tensor(vals), torch.randn(20000, generator=g) * 100,
                     torch.randn(2000, generator=g) * 1e-6])
    for dt in (torch.bfloat16, torch.float16):
        assert torch.equal(_bits(conv_ref.round_c(src, dt)), _bits(src.to(dt)))


# ----------------------------------------------------------------------------- fixtures
def test_golden_fixtures():
    """Committed vectors (tests/golden/make_golden.py) still reproduce: guards the oracle
    against silent drift."""
    path = os.path.join(GOLDEN, "golden_small.npz")
    z = np.load(path, allow_pickle=False)
    to_bf16 = lambda a: torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16)  # noqa: E731
    q, k, v = to_bf16(z["q"]), to_bf16(z["k"]), to_bf16(z["v"])
    for name, W in (("o_teacher", int(z["wt"])), ("o_student", int(z["ws"]))):
        o = attn_ref.dense_reference(q, k, v, W)
        assert np.allclose(o.numpy(), z[name], rtol=0, atol=2e-6)
    x, w = to_bf16(z["conv_x"]), to_bf16(z["conv_w"])
    assert np.array_equal(_bits(conv_ref.dwconv_c(x, w)).numpy(), z["conv_y"])


def test_golden_attn_fixtures():
    """tests/golden/golden_attn.npz (the kernels' head sizes) still reproduces: the
    oracle's fp32 outputs and LSEs."""
    sys.path.insert(0, GOLDEN)
    from make_golden import attn_cases
    z = np.load(os.path.join(GOLDEN, "golden_attn.npz"), allow_pickle=False)
    to_bf16 = lambda a: torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16)  # noqa: E731
    for name, *_ in attn_cases():
        q, k, v = (to_bf16(z[f"{name}_{t}"]) for t in "qkv")
        wt, ws = (int(w) for w in z[f"{name}_windows"])
        for which, W in (("teacher", wt), ("student", ws)):
            o, lse = attn_ref.dense_reference(q, k, v, W, return_lse=True)
            assert np.allclose(o.numpy(), z[f"{name}_o_{which}"], rtol=0, atol=2e-6)
            assert np.allclose(lse.numpy(), z[f"{name}_lse_{which}"], rtol=0, atol=2e-6)
