"""The allocation-free LSE variant (ttcd_lse_dual_window_attn_noalloc_fwd)
against the workspace entry point it is a variant of
(ttcd_lse_dual_window_attn_fwd), through the C ABI: two calls in a row, the
second on a smaller input, each bit-identical to the workspace call on the
same inputs (the first runs its far-band rows in several chunks of the fixed
64 MiB scratch, the second in one), and checked against the fp32 oracle on
sampled rows."""
from __future__ import annotations

import pytest
import torch

from oracle import attn_ref

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, HK, D, dtype, seed, dev):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g).to(dtype).to(dev)
    k = torch.randn(B, T, HK, D, generator=g).to(dtype).to(dev)
    v = torch.randn(B, T, HK, D, generator=g).to(dtype).to(dev)
    return q, k, v


def _call(q, k, v, wt, ws, noalloc):
    from ttcd_amd import _lib
    L = _lib.lib()
    B, T, H, D = q.shape
    HK = k.shape[2]
    ot = torch.empty_like(q)
    os_ = torch.empty_like(q)
    dt = _lib.DTYPE_BF16 if q.dtype == torch.bfloat16 else _lib.DTYPE_F16
    strides = (_lib.strides4(q.stride()), _lib.strides4(k.stride()), _lib.strides4(v.stride()),
               _lib.strides4(ot.stride()))
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        st = L.ttcd_lse_dual_window_attn_noalloc_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), ot.data_ptr(), os_.data_ptr(), B, T, T, H,
            HK, D, *strides, wt, ws, D ** -0.5, 8.0, dt, stream)
    else:
        nbytes = L.ttcd_lse_dual_window_attn_workspace_bytes(B, T, T, H, D, ws)
        wsb = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        st = L.ttcd_lse_dual_window_attn_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), ot.data_ptr(), os_.data_ptr(), B, T, T, H,
            HK, D, *strides, wt, ws, D ** -0.5, 8.0, dt, wsb.data_ptr(), nbytes, stream)
    _lib.check(st)
    torch.cuda.synchronize()
    return ot, os_


@torch.inference_mode()
def test_noalloc_matches_workspace_entry_two_calls(gpu):
    from ttcd_amd import _lib
    cap = _lib.lib().ttcd_lse_dual_window_attn_noalloc_scratch_bytes()
    cases = [
        # several scratch chunks: (T - ws) rows of B * H * (2D + 8) bytes exceed 64 MiB
        (4, 20000, 16, 8, 128, torch.bfloat16, 8192, 4096),
        # then a smaller call: one chunk, another head shape and dtype
        (1, 3000, 15, 5, 64, torch.float16, 1000, 500),
    ]
    for i, (B, T, H, HK, D, dtype, wt, ws) in enumerate(cases):
        print(f"noalloc case {i}: B={B} T={T} H={H} HK={HK} D={D} {dtype} wt={wt} ws={ws}",
              flush=True)
        rows_needed = (T - ws) * B * H * (2 * D + 8)
        assert (rows_needed > cap) == (i == 0)
        q, k, v = _inputs(B, T, H, HK, D, dtype, seed=11 + i, dev=gpu)
        nt, ns = _call(q, k, v, wt, ws, noalloc=True)
        rt, rs = _call(q, k, v, wt, ws, noalloc=False)
        assert torch.equal(nt, rt), f"case {i}: teacher differs from the workspace entry"
        assert torch.equal(ns, rs), f"case {i}: student differs from the workspace entry"
        # and the oracle on rows around both window edges and the end
        rows = sorted({0, ws - 1, ws, ws + 1, wt - 1, wt, wt + 7, T // 2, T - 1})
        rows = [r for r in rows if 0 <= r < T]
        b = B - 1
        qc, kc, vc = q[b:b + 1].cpu(), k[b:b + 1].cpu(), v[b:b + 1].cpu()
        for o, lo, hi in ((nt, 0, wt), (ns, 0, ws)):
            ref = attn_ref.band_reference(qc, kc, vc, lo, hi, rows=rows)
            got = o[b:b + 1, rows].float().cpu()
            err = (got - ref.float()).abs()
            assert err.max().item() <= 2e-2 and err.mean().item() <= 1e-3, (i, hi, err.max())


def _launch(q, k, v, ot, os_, wt, ws):
    """The allocation-free call on torch's current stream, no synchronisation (so it
    can be captured)."""
    from ttcd_amd import _lib
    L = _lib.lib()
    B, T, H, D = q.shape
    dt = _lib.DTYPE_BF16 if q.dtype == torch.bfloat16 else _lib.DTYPE_F16
    _lib.check(L.ttcd_lse_dual_window_attn_noalloc_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), ot.data_ptr(), os_.data_ptr(), B, T, T, H,
        k.shape[2], D, _lib.strides4(q.stride()), _lib.strides4(k.stride()),
        _lib.strides4(v.stride()), _lib.strides4(ot.stride()), wt, ws, D ** -0.5, 8.0, dt,
        torch.cuda.current_stream().cuda_stream))


@torch.inference_mode()
def test_noalloc_replays_under_graph_capture(gpu):
    """Captured in a HIP graph after one eager call on the device (which resolves the
    scratch address; the header asks for that call before any capture), three replays
    on new inputs, eager work and synchronisations between them, each bit-identical to
    the workspace entry point on the same inputs."""
    B, T, H, HK, D, wt, ws = 1, 3000, 8, 4, 128, 1500, 700
    q, k, v = _inputs(B, T, H, HK, D, torch.bfloat16, seed=21, dev=gpu)
    ot, os_ = torch.empty_like(q), torch.empty_like(q)
    _launch(q, k, v, ot, os_, wt, ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _launch(q, k, v, ot, os_, wt, ws)
    g = torch.Generator(device=gpu)
    for rep in range(3):
        g.manual_seed(200 + rep)
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, generator=g, device=gpu).to(t.dtype))
        graph.replay()
        torch.cuda.synchronize()
        got_t, got_s = ot.clone(), os_.clone()
        want_t, want_s = _call(q, k, v, wt, ws, noalloc=False)
        assert torch.equal(got_t, want_t), f"replay {rep}: teacher"
        assert torch.equal(got_s, want_s), f"replay {rep}: student"
