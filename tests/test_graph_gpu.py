"""The hot-path calls under HIP graph capture (torch.cuda.CUDAGraph).

The calls launch on torch's current stream, never synchronise and allocate
only their outputs, so a serving loop can capture them once and replay. Each
replay here runs on new inputs copied into the captured buffers, with eager
work and synchronisations between replays, and must equal the eager call on
the same inputs bit for bit."""
from __future__ import annotations

import pytest
import torch

from conftest import make_qkv

pytestmark = pytest.mark.gpu


@torch.inference_mode()
def test_hot_path_replays_equal_eager(gpu):
    from ttcd_amd import (causal_dwconv_x, epilogue, fused_dual_window_attn,
                          fused_dual_window_attn_varlen, lse_dual_window_attn, prologue)
    B, T, H, HK, D, wt, ws = 1, 1000, 8, 4, 128, 384, 130
    q, k, v = make_qkv(batch=B, seqlen=T, heads=H, kv_heads=HK, head_dim=D, seed=1)
    x = torch.randn(2, 3, 64, 256, device="cuda").to(torch.bfloat16)
    w = torch.randn(256, 5, device="cuda").to(torch.bfloat16)
    cu = torch.tensor([0, 300, 301, 1000], dtype=torch.int32, device="cuda")
    qp, kp, vp = q[0], k[0], v[0]
    wq = torch.randn(D, device="cuda").to(torch.bfloat16)
    wk = torch.randn(D, device="cuda").to(torch.bfloat16)
    cos, sin = prologue.rope_tables(prologue.rope_inv_freq(D, 1e6, "cuda"), T, torch.bfloat16)
    hid = H * D
    res = torch.randn(B, T, hid, device="cuda").to(torch.bfloat16)
    wn = torch.randn(hid, device="cuda").to(torch.bfloat16)

    def step():
        ot, os_, lt, ls = fused_dual_window_attn(q, k, v, wt, ws, return_lse=True)
        vt, vs = fused_dual_window_attn_varlen(qp, kp, vp, cu, 700, wt, ws)
        lt_, ls_ = lse_dual_window_attn(q, k, v, wt, ws)
        pq, pk = prologue.qk_norm_rope(q, k, wq, wk, 1e-6, cos, sin, 0)
        ep = epilogue.dual_residual_rmsnorm(ot.reshape(B, T, hid), os_.reshape(B, T, hid), res,
                                            wn, 1e-6)
        return (ot, os_, lt, ls, vt, vs, causal_dwconv_x(x, w), lt_, ls_, pq, pk, *ep)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm-up on a side stream, as torch's capture recipe asks
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    g = torch.Generator(device="cuda")
    for rep in range(3):
        g.manual_seed(100 + rep)
        for t in (q, k, v, x, res):
            t.copy_(torch.randn(t.shape, generator=g, device="cuda").to(t.dtype))
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        want = step()  # eager, on the same inputs
        torch.cuda.synchronize()
        for j, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a, b), f"replay {rep}, output {j}"
