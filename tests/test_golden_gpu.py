"""The GPU kernels against the committed golden vectors (tests/golden/golden_attn.npz,
written by tests/golden/make_golden.py from the CPU oracle): D=64 and D=128 at GQA
group 2, both windows truncating. The fused call (both rescale modes), the
single-band calls and the LSE variant must meet the reference's bf16 bounds
against the fp32 outputs (tests/test_attn_gpu.py) and hold their LSEs within
1e-3. (The windows are below the reference kernel's own floor, w_S >= 128 +
block_n, so no emulation of that kernel is stored; tests/test_attn_gpu.py
compares against it at config 1.)"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from test_attn_gpu import _assert_close

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
from make_golden import attn_cases  # noqa: E402


def _load(name):
    z = np.load(os.path.join(GOLDEN, "golden_attn.npz"), allow_pickle=False)
    to_bf16 = lambda a: torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16)  # noqa: E731
    q, k, v = (to_bf16(z[f"{name}_{t}"]).cuda() for t in "qkv")
    wt, ws = (int(w) for w in z[f"{name}_windows"])
    f32 = lambda key: torch.from_numpy(z[f"{name}_{key}"])  # noqa: E731
    return q, k, v, wt, ws, f32


@pytest.mark.parametrize("name", [c[0] for c in attn_cases()])
@pytest.mark.parametrize("exact", [False, True])
@torch.inference_mode()
def test_fused_matches_golden(gpu, name, exact):
    from ttcd_amd import fused_dual_window_attn
    q, k, v, wt, ws, f32 = _load(name)
    ot, os_, lt, ls = fused_dual_window_attn(q, k, v, wt, ws, return_lse=True, exact_max=exact)
    torch.cuda.synchronize()
    _assert_close(ot, f32("o_teacher"), torch.bfloat16, f"{name} teacher")
    _assert_close(os_, f32("o_student"), torch.bfloat16, f"{name} student")
    assert (lt.cpu() - f32("lse_teacher")).abs().max().item() < 1e-3
    assert (ls.cpu() - f32("lse_student")).abs().max().item() < 1e-3


@pytest.mark.parametrize("name", [c[0] for c in attn_cases()])
@torch.inference_mode()
def test_band_and_lse_variant_match_golden(gpu, name):
    from ttcd_amd import band_attn, lse_dual_window_attn
    q, k, v, wt, ws, f32 = _load(name)
    for which, W in (("teacher", wt), ("student", ws)):
        o, lse = band_attn(q, k, v, 0, W, return_lse=True)
        torch.cuda.synchronize()
        _assert_close(o, f32(f"o_{which}"), torch.bfloat16, f"{name} band {which}")
        assert (lse.cpu() - f32(f"lse_{which}")).abs().max().item() < 1e-3
    ot, os_ = lse_dual_window_attn(q, k, v, wt, ws)
    torch.cuda.synchronize()
    _assert_close(ot, f32("o_teacher"), torch.bfloat16, f"{name} LSE-variant teacher")
    _assert_close(os_, f32("o_student"), torch.bfloat16, f"{name} LSE-variant student")
