"""GPU parity of the packed-sequence (varlen) attention calls.

Every sequence of a packed batch runs the same kernel code on its own rows and
its own schedule, so each sequence's outputs and LSEs must be bit-identical to
the fixed-length call on that sequence alone (which the other GPU test files
pin against the fp32 oracle); one case is also checked against the oracle
directly. Lengths cover empty, single-token, sub-block, block-aligned and
unaligned sequences. cu_seqlens offsets past the packed rows must be clamped
(no fault, the in-range rows still correct).
"""
from __future__ import annotations

import pytest
import torch

from conftest import make_qkv, random_cases
from oracle import attn_ref

pytestmark = pytest.mark.gpu


def _packed(lens, heads, kv_heads, head_dim, seed, dtype=torch.bfloat16):
    total = sum(lens)
    q, k, v = make_qkv(batch=1, seqlen=max(total, 1), heads=heads, kv_heads=kv_heads,
                       head_dim=head_dim, dtype=dtype, seed=seed)
    q, k, v = q[0, :total], k[0, :total], v[0, :total]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32,
                      device=q.device)
    return q, k, v, cu


def _offsets(lens):
    out, s = [], 0
    for n in lens:
        out.append((s, s + n))
        s += n
    return out


LENS = [1, 127, 0, 128, 257, 700, 64, 2049]


@pytest.mark.parametrize("heads,kv_heads,head_dim,wt,ws", [
    (8, 4, 128, 512, 256),     # GQA group 2, d128
    (15, 5, 64, -1, 192),      # SmolLM2 group 3, d64, full-causal teacher
    (4, 4, 128, 1000, 999),    # MHA, narrow gap
])
@torch.inference_mode()
def test_dual_varlen_equals_per_sequence_calls(gpu, heads, kv_heads, head_dim, wt, ws):
    from ttcd_amd import fused_dual_window_attn, fused_dual_window_attn_varlen
    q, k, v, cu = _packed(LENS, heads, kv_heads, head_dim, seed=11 + heads)
    ot, os_, lt, ls = fused_dual_window_attn_varlen(q, k, v, cu, max(LENS), wt, ws,
                                                    return_lse=True)
    torch.cuda.synchronize()
    assert ot.shape == q.shape and lt.shape == (heads, q.shape[0])
    for s0, s1 in _offsets(LENS):
        if s1 == s0:
            continue
        qs, ks, vs = (t[s0:s1].unsqueeze(0) for t in (q, k, v))
        # the fixed-length wrapper asserts ws <= wt with wt = T for a full-causal
        # teacher; the kernel clamps both windows to the sequence length alike
        wt_ref = (s1 - s0) if wt < 0 else wt
        rt, rs, rlt, rls = fused_dual_window_attn(qs, ks, vs, wt_ref, min(ws, wt_ref),
                                                  return_lse=True)
        assert torch.equal(ot[s0:s1], rt[0]), (s0, s1)
        assert torch.equal(os_[s0:s1], rs[0]), (s0, s1)
        assert torch.equal(lt[:, s0:s1], rlt[0]), (s0, s1)
        assert torch.equal(ls[:, s0:s1], rls[0]), (s0, s1)


@pytest.mark.parametrize("lo,hi", [(0, 300), (128, 640)])
@torch.inference_mode()
def test_band_varlen_equals_per_sequence_calls(gpu, lo, hi):
    from ttcd_amd import band_attn, band_attn_varlen
    q, k, v, cu = _packed(LENS, 8, 4, 128, seed=5)
    o, lse = band_attn_varlen(q, k, v, cu, max(LENS), lo, hi, return_lse=True)
    torch.cuda.synchronize()
    for s0, s1 in _offsets(LENS):
        if s1 == s0:
            continue
        r, rl = band_attn(*(t[s0:s1].unsqueeze(0) for t in (q, k, v)), lo, hi, return_lse=True)
        assert torch.equal(o[s0:s1], r[0]), (s0, s1)
        assert torch.equal(lse[:, s0:s1], rl[0]), (s0, s1)


@torch.inference_mode()
def test_dual_varlen_matches_fp32_oracle(gpu):
    from ttcd_amd import fused_dual_window_attn_varlen
    lens = [300, 1, 513]
    q, k, v, cu = _packed(lens, 4, 2, 64, seed=3)
    ot, os_ = fused_dual_window_attn_varlen(q, k, v, cu, max(lens), 200, 97)
    for s0, s1 in _offsets(lens):
        qs, ks, vs = (t[s0:s1].unsqueeze(0).cpu() for t in (q, k, v))
        for W, out in ((200, ot), (97, os_)):
            ref = attn_ref.dense_reference(qs, ks, vs, W)
            mx, mean = attn_ref.error_stats(out[s0:s1].unsqueeze(0).cpu(), ref)
            assert mx <= 2e-2 and mean <= 4e-4, (s0, s1, W, mx, mean)


@torch.inference_mode()
def test_varlen_clamps_offsets_past_the_rows(gpu):
    """The last offset points past the packed rows: the sequence is clamped to them."""
    from ttcd_amd import fused_dual_window_attn, fused_dual_window_attn_varlen
    q, k, v, _ = _packed([100, 100], 4, 2, 128, seed=8)
    cu = torch.tensor([0, 100, 300], dtype=torch.int32, device=q.device)
    ot, os_ = fused_dual_window_attn_varlen(q, k, v, cu, 300, 64, 32)
    torch.cuda.synchronize()
    for s0, s1 in ((0, 100), (100, 200)):
        rt, rs = fused_dual_window_attn(*(t[s0:s1].unsqueeze(0) for t in (q, k, v)), 64, 32)
        assert torch.equal(ot[s0:s1], rt[0]) and torch.equal(os_[s0:s1], rs[0])


@torch.inference_mode()
def test_varlen_argument_checks(gpu):
    from ttcd_amd import fused_dual_window_attn_varlen
    q, k, v, cu = _packed([10, 20], 4, 2, 64, seed=1)
    with pytest.raises(ValueError):
        fused_dual_window_attn_varlen(q, k, v, cu.long(), 20, 16, 8)  # int64 offsets
    with pytest.raises(ValueError):
        fused_dual_window_attn_varlen(q.unsqueeze(0), k, v, cu, 20, 16, 8)
    with pytest.raises(ValueError):
        fused_dual_window_attn_varlen(q, k, v, cu, 0, 16, 8)
    with pytest.raises(AssertionError):
        fused_dual_window_attn_varlen(q, k, v, cu, 20, 8, 16)


def _random_varlen_case(i):
    import random
    r = random.Random(3000 + i)
    lens = [r.choice([0, 1, r.randint(1, 130), r.randint(100, 1200)]) for _ in range(r.randint(1, 6))]
    D = r.choice([64, 128])
    kv_heads = r.choice([1, 2, 4])
    heads = kv_heads * r.choice([1, 2, 3])
    mx = max(max(lens), 1)
    wt = r.choice([-1, r.randint(1, mx + 200), r.randint(1, 300)])
    ws = r.choice([1, r.randint(1, 300), wt if wt > 0 else mx])
    dtype = r.choice([torch.bfloat16, torch.float16])
    return lens, heads, kv_heads, D, wt, ws, dtype, r.random() < 0.3


@pytest.mark.parametrize("i", range(random_cases(40)))
@torch.inference_mode()
def test_random_varlen_equals_per_sequence_calls(gpu, i):
    """Seeded random packings, head shapes, windows and dtypes: every sequence
    bit-identical to the fixed-length call on it alone, in the chosen rescale mode."""
    from ttcd_amd import fused_dual_window_attn, fused_dual_window_attn_varlen
    lens, heads, kv_heads, D, wt, ws, dtype, exact = _random_varlen_case(i)
    print(f"case {i}: lens {lens} H {heads}/{kv_heads} D {D} wt {wt} ws {ws} {dtype} "
          f"exact_max {exact}", flush=True)
    q, k, v, cu = _packed(lens, heads, kv_heads, D, seed=400 + i, dtype=dtype)
    if wt > 0:
        ws = min(ws, wt)
    ot, os_, lt, ls = fused_dual_window_attn_varlen(q, k, v, cu, max(max(lens), 1), wt, ws,
                                                    return_lse=True, exact_max=exact)
    torch.cuda.synchronize()
    for s0, s1 in _offsets(lens):
        if s1 == s0:
            continue
        qs, ks, vs = (t[s0:s1].unsqueeze(0) for t in (q, k, v))
        wt_ref = (s1 - s0) if wt < 0 else wt
        rt, rs, rlt, rls = fused_dual_window_attn(qs, ks, vs, wt_ref, min(ws, wt_ref),
                                                  return_lse=True, exact_max=exact)
        assert torch.equal(ot[s0:s1], rt[0]), (i, s0, s1)
        assert torch.equal(os_[s0:s1], rs[0]), (i, s0, s1)
        assert torch.equal(lt[:, s0:s1], rlt[0]), (i, s0, s1)
        assert torch.equal(ls[:, s0:s1], rls[0]), (i, s0, s1)
