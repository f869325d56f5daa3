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
def test_dual_window_and_conv_replays_equal_eager(gpu):
    from ttcd_amd import causal_dwconv_x, fused_dual_window_attn, fused_dual_window_attn_varlen
    B, T, H, HK, D, wt, ws = 1, 1000, 8, 4, 128, 384, 130
    q, k, v = make_qkv(batch=B, seqlen=T, heads=H, kv_heads=HK, head_dim=D, seed=1)
    x = torch.randn(2, 3, 64, 256, device="cuda").to(torch.bfloat16)
    w = torch.randn(256, 5, device="cuda").to(torch.bfloat16)
    cu = torch.tensor([0, 300, 301, 1000], dtype=torch.int32, device="cuda")
    qp, kp, vp = q[0], k[0], v[0]

    def step():
        ot, os_, lt, ls = fused_dual_window_attn(q, k, v, wt, ws, return_lse=True)
        vt, vs = fused_dual_window_attn_varlen(qp, kp, vp, cu, 700, wt, ws)
        return ot, os_, lt, ls, vt, vs, causal_dwconv_x(x, w)

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
        for t in (q, k, v, x):
            t.copy_(torch.randn(t.shape, generator=g, device="cuda").to(t.dtype))
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        want = step()  # eager, on the same inputs
        torch.cuda.synchronize()
        for j, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a, b), f"replay {rep}, output {j}"
