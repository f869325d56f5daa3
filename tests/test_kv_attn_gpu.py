"""Cached prefill on the GPU: Tq new queries against Tk >= Tq keys, the
queries at the last Tq positions (flash-attention's bottom-right aligned
causal mask).

The reference specifies this case in test/test_fused_dual_attn.py:275-293
(Tq=256, Tk=384, full-causal teacher, student window 192, seed 19) and marks
it a strict xfail for its kernel. Here it must pass against the oracle, and,
since each query row's work depends only on its absolute position, the
(Tq, Tk) call must equal the last Tq rows of the full (Tk, Tk) call bit for
bit, LSEs included."""
from __future__ import annotations

import pytest
import torch

from conftest import make_qkv
from oracle import attn_ref
from test_attn_gpu import _assert_close
from ttcd_amd import band_attn, fused_dual_window_attn, lse_dual_window_attn, window_attn

pytestmark = pytest.mark.gpu


def _oracle_rows(q, k, v, lo, hi, q_off):
    """The band [lo, hi) for queries at absolute positions q_off .. Tk-1."""
    B, Tq, H, D = q.shape
    Tk = k.shape[1]
    qp = torch.zeros(B, Tk, H, D, dtype=q.dtype)
    qp[:, q_off:] = q.cpu()
    rows = torch.arange(q_off, Tk)
    return attn_ref.band_reference(qp, k.cpu(), v.cpu(), lo, hi, rows=rows)


def test_reference_xfail_case_passes(gpu):
    # test/test_fused_dual_attn.py:279-293, with the oracle in place of flash-attention
    _, k, v = make_qkv(batch=1, seqlen=384, heads=4, kv_heads=2, head_dim=64, seed=19)
    g = torch.Generator().manual_seed(19)
    q = torch.randn(1, 256, 4, 64, generator=g).to(torch.bfloat16).cuda()
    with torch.inference_mode():
        o_t, o_s = fused_dual_window_attn(q, k, v, -1, 192)
    torch.cuda.synchronize()
    _assert_close(o_t, _oracle_rows(q, k, v, 0, 384, 128), torch.bfloat16, "teacher")
    _assert_close(o_s, _oracle_rows(q, k, v, 0, 192, 128), torch.bfloat16, "student")


CASES = [
    # B, Tq, Tk, H, HK, D, wt, ws
    pytest.param(1, 256, 384, 4, 2, 64, -1, 192, id="reference-shape"),
    pytest.param(2, 300, 1000, 8, 2, 128, 512, 256, id="unaligned-offset"),
    pytest.param(1, 1, 777, 4, 4, 128, 256, 100, id="one-query"),
    pytest.param(1, 640, 640, 15, 5, 64, 512, 256, id="tq-equals-tk"),
    pytest.param(1, 129, 4096, 16, 8, 128, 2048, 1024, id="deep-cache"),
]


@pytest.mark.parametrize("B,Tq,Tk,H,HK,D,wt,ws", CASES)
def test_rows_equal_the_full_call(gpu, B, Tq, Tk, H, HK, D, wt, ws):
    qf, k, v = make_qkv(batch=B, seqlen=Tk, heads=H, kv_heads=HK, head_dim=D, seed=Tq + Tk)
    q = qf[:, Tk - Tq:].contiguous()
    with torch.inference_mode():
        ft, fs, flt, fls = fused_dual_window_attn(qf, k, v, wt, ws, return_lse=True)
        ot, os_, lt, ls = fused_dual_window_attn(q, k, v, wt, ws, return_lse=True)
        bf, blf = band_attn(qf, k, v, ws, wt if wt > 0 else Tk, return_lse=True)
        bo, bl = band_attn(q, k, v, ws, wt if wt > 0 else Tk, return_lse=True)
        wf = window_attn(qf, k, v, ws)
        wo = window_attn(q, k, v, ws)
        lt_f, ls_f = lse_dual_window_attn(qf, k, v, wt, ws) if ws < (wt if wt > 0 else Tk) \
            else (None, None)
        lt_o, ls_o = lse_dual_window_attn(q, k, v, wt, ws) if lt_f is not None else (None, None)
    torch.cuda.synchronize()
    s = slice(Tk - Tq, Tk)
    assert torch.equal(ot, ft[:, s]) and torch.equal(os_, fs[:, s])
    assert torch.equal(lt, flt[:, :, s]) and torch.equal(ls, fls[:, :, s])
    assert torch.equal(bo, bf[:, s]) and torch.equal(bl, blf[:, :, s])
    assert torch.equal(wo, wf[:, s])
    if lt_f is not None:
        assert torch.equal(lt_o, lt_f[:, s]) and torch.equal(ls_o, ls_f[:, s])
    # and against the oracle
    W = wt if wt > 0 else Tk
    _assert_close(ot, _oracle_rows(q, k, v, 0, W, Tk - Tq), torch.bfloat16, "teacher")
    _assert_close(os_, _oracle_rows(q, k, v, 0, ws, Tk - Tq), torch.bfloat16, "student")


def test_rejects_more_queries_than_keys(gpu):
    q, k, v = make_qkv(batch=1, seqlen=256, heads=2, kv_heads=2, head_dim=64)
    with pytest.raises(ValueError):
        fused_dual_window_attn(q, k[:, :128], v[:, :128], 64, 32)
