"""The lazy slot of the D = 128 kernel (ttcd_amd/csrc/attn.hip: slot_body_lazy)
on inputs that drive its rescue path in many tiles.

Its rule: a row keeps its reference max until a 64-key tile's probabilities
against it sum above 2^rescale_log2 over a half row (32 keys), or until the row
has its first unmasked keys; that tile then takes the row max, moves the
reference of the rows out of bound and redoes its exp2. On N(0,1) inputs this
happens in the first tile of a row and rarely after. Here the keys are scaled
up with their distance from the end of the sequence, so the sweep (from the
diagonal backwards) meets a higher row max tile after tile and takes the rescue
path over and over. Checked against the fp32 oracle, outputs and LSEs, in bf16
and in f16 at the largest bound the ABI allows for f16 (2^15, through the C
ABI), for the fused dual-window call, the single-band call and the exact mode.
"""
from __future__ import annotations

import pytest
import torch

from conftest import make_qkv
from oracle import attn_ref
from test_attn_random_gpu import _assert_close

pytestmark = pytest.mark.gpu


def _rising_qkv(T, H, HK, dtype, seed, growth):
    q, k, v = make_qkv(batch=1, seqlen=T, heads=H, kv_heads=HK, head_dim=128, dtype=dtype,
                       seed=seed, device="cpu")
    j = torch.arange(T, dtype=torch.float32)
    scale = 1.0 + growth * (T - 1 - j) / T
    k = (k.float() * scale.view(1, T, 1, 1)).to(dtype)
    return q.cuda(), k.cuda(), v.cuda()


def _check(out, lse, q, k, v, W, dtype, what, lo=0):
    ro, rl = attn_ref.dense_reference(q.cpu(), k.cpu(), v.cpu(), W, lo=lo, return_lse=True)
    _assert_close(out, ro, dtype, what)
    rl = rl.float()
    fin = torch.isfinite(rl)
    assert torch.equal(torch.isfinite(lse.cpu()), fin), f"{what}: lse finiteness"
    d = (lse.cpu()[fin] - rl[fin]).abs() / rl[fin].abs().clamp(min=1.0)
    assert d.max().item() < 1e-4, f"{what}: lse rel err {d.max().item():.3g}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("wt,ws", [(-1, 300), (700, 128), (1100, 1099), (64, 1)])
@pytest.mark.parametrize("growth", [2.0, 5.0])
@torch.inference_mode()
def test_rising_scores_fused(gpu, dtype, wt, ws, growth):
    from ttcd_amd import fused_dual_window_attn
    T = 1200
    q, k, v = _rising_qkv(T, 4, 2, dtype, seed=int(growth * 10) + ws, growth=growth)
    W = T if wt < 0 else wt
    for exact in (False, True):
        ot, os_, lt, ls = fused_dual_window_attn(q, k, v, wt, ws, return_lse=True, exact_max=exact)
        tag = f"{'exact' if exact else 'lazy'} growth={growth}"
        _check(ot, lt, q, k, v, W, dtype, f"teacher {tag}")
        _check(os_, ls, q, k, v, ws, dtype, f"student {tag}")


@pytest.mark.parametrize("lo,hi", [(0, 500), (200, 900), (1, 2)])
@torch.inference_mode()
def test_rising_scores_band(gpu, lo, hi):
    from ttcd_amd import band_attn
    T = 1000
    q, k, v = _rising_qkv(T, 6, 3, torch.bfloat16, seed=lo + hi, growth=4.0)
    o, lse = band_attn(q, k, v, lo, hi, return_lse=True)
    ro, rl = attn_ref.dense_reference(q.cpu(), k.cpu(), v.cpu(), hi, lo=lo, return_lse=True)
    empty = torch.isinf(rl.float())
    assert torch.equal(torch.isinf(lse.cpu()), empty)
    o_rows = o.float().cpu().permute(0, 2, 1, 3)
    assert (o_rows[empty] == 0).all()
    _assert_close(o, ro, torch.bfloat16, f"band {lo},{hi}")


@pytest.mark.parametrize("rescale_log2", [15.0, 1.0])
@torch.inference_mode()
def test_f16_largest_bound_through_c_abi(gpu, rescale_log2):
    """f16 at rescale_log2 = 15: probabilities reach up to 2^15 before they are
    rounded to f16 (max 65504), so nothing overflows; 1.0 rescues in almost
    every tile."""
    from ttcd_amd import _lib
    L = _lib.lib()
    T, H, HK, D, wt, ws = 1100, 4, 2, 128, 800, 200
    q, k, v = _rising_qkv(T, H, HK, torch.float16, seed=15, growth=5.0)
    ot = torch.empty_like(q)
    os_ = torch.empty_like(q)
    lt = torch.empty(1, H, T, device=q.device, dtype=torch.float32)
    ls = torch.empty_like(lt)
    _lib.check(L.ttcd_dual_window_attn_kv_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), ot.data_ptr(), os_.data_ptr(), lt.data_ptr(),
        ls.data_ptr(), 1, T, T, H, HK, D, _lib.strides4(q.stride()), _lib.strides4(k.stride()),
        _lib.strides4(v.stride()), _lib.strides4(ot.stride()), wt, ws, D ** -0.5, rescale_log2,
        _lib.DTYPE_F16, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    _check(ot, lt, q, k, v, wt, torch.float16, f"teacher f16 rescale_log2={rescale_log2}")
    _check(os_, ls, q, k, v, ws, torch.float16, f"student f16 rescale_log2={rescale_log2}")
