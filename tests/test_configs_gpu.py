"""The BASELINE workloads beyond the headline, run at their full size on the
GPU and checked against the fp32 oracle on sampled rows (the oracle's banded
form evaluates any subset of rows at the cost of those rows alone):

* config 3, SmolLM2-360M's layer: T=65536, Hq=15, Hkv=5 (GQA group 3),
  D=64, (w_T, w_S) = (8192, 4096) (configs/ipttcd/
  ipttcdv9_smollm2_360M_ct_64k_v2_swa8k.json:3-12);
* config 4, the batch and narrow-gap sweep at the Qwen3-0.6B head shape:
  B=8 at T=16384 with (8192, 4096), and T=32768 with the narrow gaps
  (8192, 7168) and (8192, 8064), where the teacher window truncates, so the
  far band's lower edge and its masking run on the GPU
  (profiling/bench_attn_bsz.py:26-40);
* the LSE-combination variant on the same shapes, since config 4 compares it
  with the fused kernel;
* a sequence four times the headline length (T=262144) at both head sizes.

Outputs and LSEs are checked on rows around 0, w_S, w_T and the tail, at the
attention bars of test_attn_gpu.py; size-independent properties (finite
outputs, teacher == student below w_S) are checked on every row.
"""
from __future__ import annotations

import pytest
import torch

from conftest import make_qkv
from oracle import attn_ref
from test_attn_gpu import _assert_close

pytestmark = pytest.mark.gpu


def _rows(T, wt, ws, extra=()):
    parts = [torch.arange(0, 48), torch.arange(ws - 40, ws + 40), torch.arange(wt - 40, wt + 72),
             torch.arange(T - 48, T)] + [torch.arange(a, a + 32) for a in extra]
    return torch.cat(parts).clamp(0, T - 1).unique()


def _check_sampled(q, k, v, outs, wt, ws, rows, batches, dtype):
    """outs = (o_t, o_s, lse_t, lse_s); every listed batch entry on `rows`."""
    ot, os_, lt, ls = outs
    for b in batches:
        qc, kc, vc = q[b:b + 1].cpu(), k[b:b + 1].cpu(), v[b:b + 1].cpu()
        for W, o, lse in ((wt, ot, lt), (ws, os_, ls)):
            ro, rl = attn_ref.band_reference(qc, kc, vc, 0, W, rows=rows, return_lse=True)
            _assert_close(o[b:b + 1, rows], ro, dtype, f"b={b} W={W}")
            if lse is not None:
                d = (lse[b:b + 1, :, rows].cpu() - rl).abs().max().item()
                assert d < 1e-3, f"b={b} W={W}: lse max err {d:.3g}"


@torch.inference_mode()
def test_config3_smollm2_64k(gpu):
    from ttcd_amd import fused_dual_window_attn
    T, WT, WS = 65536, 8192, 4096
    print("config 3: SmolLM2 T=65536 Hq=15 Hkv=5 D=64 (8192, 4096)", flush=True)
    q, k, v = make_qkv(batch=1, seqlen=T, heads=15, kv_heads=5, head_dim=64, seed=3)
    outs = fused_dual_window_attn(q, k, v, WT, WS, return_lse=True)
    torch.cuda.synchronize()
    ot, os_ = outs[0], outs[1]
    assert ot.isfinite().all() and os_.isfinite().all()
    assert torch.equal(ot[:, :WS], os_[:, :WS])
    _check_sampled(q, k, v, outs, WT, WS, _rows(T, WT, WS, extra=(30000, 50001)), [0],
                   torch.bfloat16)


@torch.inference_mode()
def test_config3_smollm2_64k_lse_variant(gpu):
    from ttcd_amd import lse_dual_window_attn
    T, WT, WS = 65536, 8192, 4096
    q, k, v = make_qkv(batch=1, seqlen=T, heads=15, kv_heads=5, head_dim=64, seed=5)
    ot, os_ = lse_dual_window_attn(q, k, v, WT, WS)
    torch.cuda.synchronize()
    assert ot.isfinite().all() and torch.equal(ot[:, :WS], os_[:, :WS])
    _check_sampled(q, k, v, (ot, os_, None, None), WT, WS, _rows(T, WT, WS), [0],
                   torch.bfloat16)


@torch.inference_mode()
def test_config4_batch8_16k(gpu):
    from ttcd_amd import fused_dual_window_attn, lse_dual_window_attn
    B, T, WT, WS = 8, 16384, 8192, 4096
    print("config 4: B=8 T=16384 Hq=16 Hkv=8 D=128 (8192, 4096)", flush=True)
    q, k, v = make_qkv(batch=B, seqlen=T, heads=16, kv_heads=8, head_dim=128, seed=8)
    outs = fused_dual_window_attn(q, k, v, WT, WS, return_lse=True)
    torch.cuda.synchronize()
    ot, os_ = outs[0], outs[1]
    assert ot.isfinite().all() and os_.isfinite().all()
    assert torch.equal(ot[:, :WS], os_[:, :WS])
    rows = _rows(T, WT, WS, extra=(12000,))
    _check_sampled(q, k, v, outs, WT, WS, rows, [0, 5, 7], torch.bfloat16)
    # batch entries are independent: entry 5 alone gives the same bits
    one = fused_dual_window_attn(q[5:6], k[5:6], v[5:6], WT, WS, return_lse=True)
    for a, b in zip(outs, one):
        assert torch.equal(a[5:6], b)
    lt, ls = lse_dual_window_attn(q, k, v, WT, WS)
    torch.cuda.synchronize()
    _check_sampled(q, k, v, (lt, ls, None, None), WT, WS, rows, [7], torch.bfloat16)


@pytest.mark.parametrize("ws", [7168, 8064])
@torch.inference_mode()
def test_config4_narrow_gaps_32k(gpu, ws):
    """T = 32768 > w_T: the teacher window truncates, so rows past w_T fold a
    far band whose lower edge moves with the row. Rows around w_T - 1 ..
    w_T + 64 (first truncated rows), around w_S and the tail."""
    from ttcd_amd import fused_dual_window_attn, lse_dual_window_attn
    T, WT = 32768, 8192
    print(f"config 4: T=32768 narrow gap (8192, {ws})", flush=True)
    q, k, v = make_qkv(batch=1, seqlen=T, heads=16, kv_heads=8, head_dim=128, seed=ws)
    outs = fused_dual_window_attn(q, k, v, WT, ws, return_lse=True)
    torch.cuda.synchronize()
    assert outs[0].isfinite().all() and outs[1].isfinite().all()
    assert torch.equal(outs[0][:, :ws], outs[1][:, :ws])
    rows = _rows(T, WT, ws, extra=(WT + ws, 20000))
    _check_sampled(q, k, v, outs, WT, ws, rows, [0], torch.bfloat16)
    lt, ls = lse_dual_window_attn(q, k, v, WT, ws)
    torch.cuda.synchronize()
    _check_sampled(q, k, v, (lt, ls, None, None), WT, ws, rows, [0], torch.bfloat16)


@pytest.mark.parametrize("wt,ws", [(8192, 7168), (8192, 8064), (4224, 4096)])
@torch.inference_mode()
def test_narrow_gaps_with_active_teacher_boundary(gpu, wt, ws):
    """The narrow-gap windows at T = w_T + 384 (not only T = w_T), smaller
    heads, fp16: the rows just past w_T are checked against the oracle."""
    from ttcd_amd import fused_dual_window_attn
    T = wt + 384
    q, k, v = make_qkv(batch=1, seqlen=T, heads=4, kv_heads=2, head_dim=128, seed=wt - ws,
                       dtype=torch.float16)
    outs = fused_dual_window_attn(q, k, v, wt, ws, return_lse=True)
    torch.cuda.synchronize()
    rows = torch.cat([torch.arange(wt - 8, T), torch.arange(ws - 16, ws + 16)]).unique()
    _check_sampled(q, k, v, outs, wt, ws, rows, [0], torch.float16)


@pytest.mark.parametrize("heads,kv_heads,head_dim", [(2, 1, 128), (3, 1, 64)])
@torch.inference_mode()
def test_long_sequence_256k(gpu, heads, kv_heads, head_dim):
    """T = 262144, four times the headline length (query blocks, slot words
    and element offsets at that size), both head sizes, the even (two heads
    per wavefront) and odd group layouts; rows around 0, w_S, w_T, the
    middle and the tail against the oracle."""
    from ttcd_amd import fused_dual_window_attn
    T, WT, WS = 262144, 8192, 4096
    print(f"long sequence: T={T} Hq={heads} Hkv={kv_heads} D={head_dim}", flush=True)
    q, k, v = make_qkv(batch=1, seqlen=T, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
                       seed=head_dim + heads)
    outs = fused_dual_window_attn(q, k, v, WT, WS, return_lse=True)
    torch.cuda.synchronize()
    assert outs[0].isfinite().all() and outs[1].isfinite().all()
    assert torch.equal(outs[0][:, :WS], outs[1][:, :WS])
    rows = _rows(T, WT, WS, extra=(131000, 200003))
    _check_sampled(q, k, v, outs, WT, WS, rows, [0], torch.bfloat16)
