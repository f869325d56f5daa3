"""GPU parity of the LSE-combination variant (profiling/lse_dual_attn.py) and of the
single-band kernel it is built from, against the fp32 CPU oracle."""
from __future__ import annotations

import pytest
import torch

from conftest import make_qkv
from oracle import attn_ref
from test_attn_gpu import _assert_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fn", ["lse_dual_window_attn", "lse_dual_window_attn_fa3",
                                "lse_dual_window_attn_fa3_fast"])
@pytest.mark.parametrize("T,H,HK,D,wt,ws", [(769, 8, 4, 128, 512, 256), (513, 15, 5, 64, -1, 256),
                                            (600, 4, 4, 64, 300, 299)])
@torch.inference_mode()
def test_lse_variant_matches_oracle(gpu, fn, T, H, HK, D, wt, ws):
    import ttcd_amd
    q, k, v = make_qkv(batch=1, seqlen=T, heads=H, kv_heads=HK, head_dim=D, seed=7)
    ot, os_ = getattr(ttcd_amd, fn)(q, k, v, wt, ws)
    _assert_close(ot, attn_ref.dense_reference(q.cpu(), k.cpu(), v.cpu(), wt), q.dtype, "teacher")
    _assert_close(os_, attn_ref.dense_reference(q.cpu(), k.cpu(), v.cpu(), ws), q.dtype, "student")
    # the student is exactly the single-window call; the first WS teacher rows copy it
    assert torch.equal(os_, ttcd_amd.window_attn(q, k, v, ws))
    assert torch.equal(ot[:, :ws], os_[:, :ws])


@torch.inference_mode()
def test_lse_variant_short_sequence_returns_student_twice(gpu):
    import ttcd_amd
    q, k, v = make_qkv(batch=1, seqlen=100, heads=4, kv_heads=2, head_dim=64, seed=1)
    ot, os_ = ttcd_amd.lse_dual_window_attn(q, k, v, 512, 256)
    assert ot is os_


def test_lse_variant_requires_strict_gap(gpu):
    import ttcd_amd
    q, k, v = make_qkv(batch=1, seqlen=100, heads=4, kv_heads=2, head_dim=64, seed=1)
    with pytest.raises(AssertionError):
        ttcd_amd.lse_dual_window_attn(q, k, v, 256, 256)


@pytest.mark.parametrize("lo,hi", [(0, 1), (0, 77), (64, 300), (199, 200), (5, 10**6), (700, 900)])
@torch.inference_mode()
def test_band_kernel(gpu, lo, hi):
    from ttcd_amd import band_attn
    q, k, v = make_qkv(batch=2, seqlen=640, heads=6, kv_heads=3, head_dim=128, seed=lo + 3)
    o, lse = band_attn(q, k, v, lo, hi, return_lse=True)
    ro, rl = attn_ref.dense_reference(q.cpu(), k.cpu(), v.cpu(), hi, lo=lo, return_lse=True)
    _assert_close(o, ro, torch.bfloat16, f"band {lo},{hi}")
    rl = rl.float()
    empty = torch.isinf(rl)
    assert torch.equal(torch.isinf(lse.cpu()), empty)
    assert (lse.cpu()[~empty] - rl[~empty]).abs().max().item() < 1e-3 if (~empty).any() else True
    assert (o.float().cpu().permute(0, 2, 1, 3)[empty] == 0).all()


@torch.inference_mode()
def test_merge_kernel(gpu):
    from ttcd_amd import lse_merge
    g = torch.Generator().manual_seed(3)
    B, T, H, D = 2, 333, 5, 64
    o_s = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16)
    o_f = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16)
    l_s = torch.randn(B, H, T, generator=g) * 3
    l_f = torch.randn(B, H, T, generator=g) * 3
    l_f[:, :, 100:110] = float("-inf")
    out = lse_merge(o_s.cuda(), l_s.cuda(), o_f.cuda(), l_f.cuda(), row_start=50).cpu()
    ref, _ = attn_ref.lse_merge_reference(o_s, l_s, o_f, l_f)
    ref = ref.to(torch.bfloat16)
    assert torch.equal(out[:, :50], o_s[:, :50])
    assert torch.equal(out[:, 100:110], o_s[:, 100:110])
    rep = attn_ref.ulp_report(out[:, 50:], ref[:, 50:])
    assert rep["max_ulp"] <= 1 and rep["bit_equal_pct"] > 97.0, rep


def lse_variant_c(q, k, v, wt, ws, workspace_bytes=None, exact_max=False):
    """ttcd_lse_dual_window_attn_fwd through the C ABI with a workspace of
    `workspace_bytes` (None: the one-pass size)."""
    from ttcd_amd import _lib
    L = _lib.lib()
    B, Tq, H, D = q.shape
    Tk, HK = k.shape[1], k.shape[2]
    need = L.ttcd_lse_dual_window_attn_workspace_bytes(B, Tq, Tk, H, D, ws)
    nbytes = need if workspace_bytes is None else workspace_bytes
    wsb = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    ot = torch.empty_like(q)
    os_ = torch.empty_like(q)
    dt = _lib.DTYPE_BF16 if q.dtype == torch.bfloat16 else _lib.DTYPE_F16
    _lib.check(L.ttcd_lse_dual_window_attn_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), ot.data_ptr(), os_.data_ptr(), B, Tq, Tk, H, HK,
        D, _lib.strides4(q.stride()), _lib.strides4(k.stride()), _lib.strides4(v.stride()),
        _lib.strides4(ot.stride()), wt, ws, D ** -0.5, 0.0 if exact_max else 8.0, dt,
        wsb.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream))
    return ot, os_, need


@pytest.mark.parametrize("B,Tq,Tk,H,HK,D,wt,ws,dtype", [
    (1, 1500, 1500, 8, 4, 128, 700, 300, torch.bfloat16),
    (2, 1000, 1000, 15, 5, 64, -1, 257, torch.float16),
    (1, 700, 1300, 4, 2, 128, 900, 128, torch.bfloat16),   # cached prefill, Tq < Tk
    (3, 333, 333, 6, 3, 64, 200, 199, torch.bfloat16),
])
@torch.inference_mode()
def test_lse_variant_chunked_workspace_is_bitwise(gpu, B, Tq, Tk, H, HK, D, wt, ws, dtype):
    """A workspace smaller than the one-pass size runs the far-band rows in
    chunks; every row's result depends only on its absolute position, so the
    outputs are bit-identical to the one-pass call, and the one-pass call
    matches the oracle."""
    g = torch.Generator().manual_seed(B * 1000 + Tq)
    q = torch.randn(B, Tq, H, D, generator=g).to(dtype).to(gpu)
    k = torch.randn(B, Tk, HK, D, generator=g).to(dtype).to(gpu)
    v = torch.randn(B, Tk, HK, D, generator=g).to(dtype).to(gpu)
    ot, os_, need = lse_variant_c(q, k, v, wt, ws)
    per_row = B * H * (2 * D + 8)
    for rows in (1, 100, 300):
        ct, cs, _ = lse_variant_c(q, k, v, wt, ws, workspace_bytes=rows * per_row + 768)
        assert torch.equal(ct, ot) and torch.equal(cs, os_), rows
    W = Tk if wt < 0 else wt
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    # the oracle aligns the Tq queries bottom-right against the Tk keys
    rt = attn_ref.dense_reference(qc, kc, vc, W)
    rs = attn_ref.dense_reference(qc, kc, vc, ws)
    _assert_close(ot, rt, dtype, "teacher")
    _assert_close(os_, rs, dtype, "student")
    assert torch.equal(os_, __import__("ttcd_amd").window_attn(q, k, v, ws))
