"""The two-heads-per-wavefront geometry of the attention kernels.

For an even GQA group a wavefront holds 16 rows of each of two query heads that
share a K/V head (a workgroup spans 64 tokens); otherwise 32 rows of one head
(128 tokens). Tile boundaries are the same in both geometries and each row's
arithmetic depends on its own scores only, so a grouped call must equal, bit
for bit, one call per query head against its K/V head (group size 1: the
single-head geometry). The per-head calls are pinned against the fp32 oracle by
the other GPU test files; this file pins the grouped geometry to them, through
the fused call (both rescale modes, with LSEs), the single-band call, cached
prefill, the LSE variant and packed sequences.
"""
from __future__ import annotations

import pytest
import torch

from conftest import make_qkv

pytestmark = pytest.mark.gpu

CASES = [
    # batch, seqlen, heads, kv_heads, head_dim, dtype, wt, ws
    pytest.param(2, 1000, 4, 2, 128, torch.bfloat16, 512, 200, id="g2-d128-bf16"),
    pytest.param(1, 777, 8, 2, 64, torch.float16, -1, 300, id="g4-d64-f16-causal"),
    pytest.param(1, 4100, 2, 1, 128, torch.bfloat16, 4096, 4064, id="g2-narrow-gap-two-mixed-tiles"),
    pytest.param(1, 2500, 16, 2, 128, torch.float16, 1100, 1, id="g8-window-one"),
    pytest.param(3, 200, 4, 2, 64, torch.bfloat16, 150, 97, id="g2-short"),
]


def _per_head(fn, q, k, v, *args, **kw):
    """fn called once per query head h on (q[:, :, h], k/v[:, :, h // G]); outputs
    stacked back along the head axis (outputs: (B, T, H, D); LSEs: (B, H, T))."""
    H, HK = q.shape[2], k.shape[2]
    G = H // HK
    outs = [fn(q[:, :, h:h + 1], k[:, :, h // G:h // G + 1], v[:, :, h // G:h // G + 1], *args,
               **kw) for h in range(H)]
    if torch.is_tensor(outs[0]):
        outs = [(o,) for o in outs]
    res = []
    for i, o in enumerate(outs[0]):
        res.append(torch.cat([x[i] for x in outs], dim=2 if o.dim() == 4 else 1))
    return tuple(res)


def _assert_bitwise(got, want, what):
    for i, (a, b) in enumerate(zip(got, want)):
        assert a.shape == b.shape, (what, i, a.shape, b.shape)
        assert torch.equal(a, b), (f"{what}: output {i} differs in "
                                   f"{(a != b).sum().item()} of {a.numel()} values")


@pytest.mark.parametrize("batch,seqlen,heads,kv_heads,head_dim,dtype,wt,ws", CASES)
@pytest.mark.parametrize("exact", [False, True])
@torch.inference_mode()
def test_grouped_fused_call_equals_per_head_calls(gpu, batch, seqlen, heads, kv_heads,
                                                  head_dim, dtype, wt, ws, exact):
    from ttcd_amd import fused_dual_window_attn
    q, k, v = make_qkv(batch=batch, seqlen=seqlen, heads=heads, kv_heads=kv_heads,
                       head_dim=head_dim, dtype=dtype, seed=seqlen + heads)
    got = fused_dual_window_attn(q, k, v, wt, ws, return_lse=True, exact_max=exact)
    want = _per_head(fused_dual_window_attn, q, k, v, wt, ws, return_lse=True, exact_max=exact)
    _assert_bitwise(got, want, "fused")
    # cached prefill: the last rows of the same call
    tq = seqlen // 3 + 5
    got = fused_dual_window_attn(q[:, -tq:], k, v, wt, ws, return_lse=True, exact_max=exact)
    want = _per_head(lambda qq, kk, vv: fused_dual_window_attn(qq[:, -tq:], kk, vv, wt, ws,
                                                               return_lse=True,
                                                               exact_max=exact), q, k, v)
    _assert_bitwise(got, want, "cached prefill")


@pytest.mark.parametrize("batch,seqlen,heads,kv_heads,head_dim,dtype,wt,ws", CASES)
@torch.inference_mode()
def test_grouped_band_and_lse_calls_equal_per_head_calls(gpu, batch, seqlen, heads, kv_heads,
                                                         head_dim, dtype, wt, ws):
    from ttcd_amd import band_attn, lse_dual_window_attn
    q, k, v = make_qkv(batch=batch, seqlen=seqlen, heads=heads, kv_heads=kv_heads,
                       head_dim=head_dim, dtype=dtype, seed=seqlen + heads + 1)
    hi = seqlen if wt < 0 else wt
    for lo in (0, ws):
        if lo >= hi:
            continue
        got = band_attn(q, k, v, lo, hi, return_lse=True)
        want = _per_head(band_attn, q, k, v, lo, hi, return_lse=True)
        _assert_bitwise(got, want, f"band ({lo}, {hi})")
    if ws < hi:
        got = lse_dual_window_attn(q, k, v, wt, ws)
        want = _per_head(lse_dual_window_attn, q, k, v, wt, ws)
        _assert_bitwise(got, want, "LSE variant")


@pytest.mark.parametrize("heads,kv_heads,head_dim", [(8, 4, 128), (8, 2, 64)])
@torch.inference_mode()
def test_grouped_varlen_call_equals_per_head_calls(gpu, heads, kv_heads, head_dim):
    from ttcd_amd import fused_dual_window_attn_varlen
    lens = [1, 127, 0, 128, 300, 65, 1030]
    total = sum(lens)
    q, k, v = make_qkv(batch=1, seqlen=total, heads=heads, kv_heads=kv_heads,
                       head_dim=head_dim, seed=total)
    q, k, v = q[0], k[0], v[0]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32,
                      device=q.device)
    got = fused_dual_window_attn_varlen(q, k, v, cu, max(lens), 500, 129, return_lse=True)
    G = heads // kv_heads
    outs = [fused_dual_window_attn_varlen(q[:, h:h + 1], k[:, h // G:h // G + 1],
                                          v[:, h // G:h // G + 1], cu, max(lens), 500, 129,
                                          return_lse=True) for h in range(heads)]
    want = (torch.cat([o[0] for o in outs], dim=1), torch.cat([o[1] for o in outs], dim=1),
            torch.cat([o[2] for o in outs], dim=0), torch.cat([o[3] for o in outs], dim=0))
    _assert_bitwise(got, want, "varlen")
