"""CPU oracle for dual-window attention (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker. Everything runs in torch on the CPU in fp32 (or
fp64 where stated), except band_reference_blocked, which runs plain torch
fp32 ops on whatever device its inputs live on (the GPU tests give it GPU
tensors to check every row of the 64K shapes); none of it calls this
repository's HIP library.

Functions and the reference lines they restate
  dense_reference               - test/test_fused_dual_attn.py:88-110 (fp32
                                  einsum, repeat_interleave GQA, bottom-right
                                  alignment, mask 0 <= i - j < W, softmax), with
                                  an optional band lower bound and natural-log LSE.
  band_reference                - the same math query-chunked over the band
                                  (keys i-hi+1 .. i-lo only), optionally on a
                                  subset of rows; the form used at T = 64K.
  band_reference_blocked        - the same math again, blocked over all rows
                                  with torch.matmul (device-agnostic).
  lse_merge_reference           - profiling/lse_dual_attn.py:32-38 / :119-131.
  emulate_reference_kernel      - the block algorithm of _fused_dual_swa_fwd
                                  (profiling/fused_dual_attn.py:56-241): 64-row
                                  query blocks, 64-key blocks from the diagonal
                                  backward, segments A-E / narrow-gap segment,
                                  raw-domain max, exp2(s*c - m*c), the -inf guard,
                                  P rounded to the input dtype, reciprocal epilogue.
  ulp_report                    - profiling/fused_dual_attn.py:275-286 metric.
  brute_force_attention         - scalar float64 loops, tiny inputs only.

Pins (tests/test_oracle.py): brute_force_attention on tiny shapes (an
implementation with no shared code); closed forms (all-equal scores -> mean
of V over the window; window 1 -> o = v; window >= T -> plain causal);
dense == banded == blocked; lse == logsumexp identity; merge(student, far band) ==
teacher; the emulator against dense_reference within bf16 tolerance.
"""
from __future__ import annotations

import math

import torch

LOG2E = 1.4426950408889634
NEG_INF = float("-inf")


# --------------------------------------------------------------------------- counts
# --------------------------------------------------------------------------- references
def _norm_window(W, T):
    return T if (W is None or W < 0) else W


def dense_reference(q, k, v, window, *, lo: int = 0, return_lse: bool = False,
                    dtype=torch.float32):
    """fp32 masked softmax attention, FlashAttention bottom-right alignment.

    q (B, Tq, H, D), k/v (B, Tk, HK, D). Key j visible to query i iff
    lo <= (i + Tk - Tq) - j < window. Returns the unrounded output
    (B, Tq, H, D) in `dtype` (and lse (B, H, Tq), natural log, -inf for an
    empty row, whose output is 0).
    """
    B, Tq, H, D = q.shape
    Tk, HK = k.shape[1], k.shape[2]
    assert H % HK == 0
    W = _norm_window(window, Tk)
    kr = k.repeat_interleave(H // HK, dim=2).to(dtype)
    vr = v.repeat_interleave(H // HK, dim=2).to(dtype)
    s = torch.einsum("bqhd,bkhd->bhqk", q.to(dtype), kr) / math.sqrt(D)
    qpos = torch.arange(Tq)[:, None] + Tk - Tq
    kpos = torch.arange(Tk)[None, :]
    dist = qpos - kpos
    mask = (dist >= lo) & (dist < W)
    s = s.masked_fill(~mask[None, None], NEG_INF)
    lse = torch.logsumexp(s, dim=-1)
    p = torch.softmax(s, dim=-1).nan_to_num(0.0)
    o = torch.einsum("bhqk,bkhd->bqhd", p, vr)
    return (o, lse) if return_lse else o


def band_reference(q, k, v, lo: int, hi: int | None, *, rows=None, chunk: int = 256,
                   dtype=torch.float32, return_lse: bool = False):
    """Same math as dense_reference (Tq == Tk) computed one query chunk at a time
    over only the keys of the band [i - hi + 1, i - lo].

    rows: optional 1-D index tensor of query rows to evaluate (sorted); the
    result then has len(rows) rows. Rows with an empty band get o = 0,
    lse = -inf.
    """
    B, T, H, D = q.shape
    HK = k.shape[2]
    G = H // HK
    hi = T if (hi is None or hi < 0) else hi
    rows = torch.arange(T) if rows is None else torch.as_tensor(rows).sort().values
    n = rows.numel()
    out = torch.zeros(B, n, H, D, dtype=dtype)
    lse = torch.full((B, H, n), NEG_INF, dtype=dtype)
    scale = 1.0 / math.sqrt(D)
    start = 0
    while start < n:
        stop = start
        while stop < n and int(rows[stop]) - int(rows[start]) < chunk:
            stop += 1
        r = rows[start:stop]
        i0, i1 = int(r[0]), int(r[-1])
        jlo, jhi = max(0, i0 - hi + 1), min(T - 1, i1 - lo)
        if jhi >= jlo:
            qs = q[:, r].to(dtype).reshape(B, -1, HK, G, D)
            ks = k[:, jlo:jhi + 1].to(dtype)
            vs = v[:, jlo:jhi + 1].to(dtype)
            s = torch.einsum("bnhgd,bmhd->bhgnm", qs, ks) * scale
            dist = r[:, None] - torch.arange(jlo, jhi + 1)[None, :]
            mask = (dist >= lo) & (dist < hi)
            s = s.masked_fill(~mask, NEG_INF)
            lc = torch.logsumexp(s, dim=-1)  # (B, HK, G, n)
            p = torch.softmax(s, dim=-1).nan_to_num(0.0)
            oc = torch.einsum("bhgnm,bmhd->bnhgd", p, vs)
            out[:, start:stop] = oc.reshape(B, -1, H, D)
            lse[:, :, start:stop] = lc.reshape(B, H, -1)
        start = stop
    return (out, lse) if return_lse else out


def band_reference_blocked(q, k, v, lo: int, hi: int | None, *, q_block: int = 512,
                           return_lse: bool = False):
    """Every row of band_reference's math (Tq == Tk; fp32 masked softmax over the
    keys i-hi+1 .. i-lo of query i), a block of q_block query rows at a time, on
    the inputs' own device: contiguous fp32 operands through torch.matmul, the
    query heads of one K/V head stacked as rows (head h reads K/V head h // G).

    This is the full-size checker: on GPU tensors it evaluates all 65536 rows of
    the 64K shapes in seconds with torch's own fp32 GEMMs and softmax, a path
    that shares no code with this repository's HIP library. Returns fp32
    o (B, T, H, D) (and lse (B, H, T), natural log; -inf and o = 0 for an empty
    band).
    """
    B, T, H, D = q.shape
    HK = k.shape[2]
    G = H // HK
    hi = T if (hi is None or hi < 0) else hi
    dev = q.device
    out = torch.zeros(B, T, H, D, dtype=torch.float32, device=dev)
    lse = torch.full((B, H, T), NEG_INF, dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(D)
    for i0 in range(0, T, q_block):
        i1 = min(T, i0 + q_block)
        jlo, jhi = max(0, i0 - hi + 1), min(T - 1, i1 - 1 - lo)
        if jhi < jlo:
            continue
        n, m = i1 - i0, jhi - jlo + 1
        qs = (q[:, i0:i1].float().reshape(B, n, HK, G, D).permute(0, 2, 3, 1, 4)
              .reshape(B, HK, G * n, D).contiguous())
        ks_t = k[:, jlo:jhi + 1].float().permute(0, 2, 3, 1).contiguous()  # (B, HK, D, m)
        vs = v[:, jlo:jhi + 1].float().permute(0, 2, 1, 3).contiguous()    # (B, HK, m, D)
        s = torch.matmul(qs, ks_t).mul_(scale).view(B, HK, G, n, m)
        dist = (torch.arange(i0, i1, device=dev)[:, None]
                - torch.arange(jlo, jhi + 1, device=dev)[None, :])
        s.masked_fill_(~((dist >= lo) & (dist < hi)), NEG_INF)
        lc = torch.logsumexp(s, dim=-1)  # (B, HK, G, n)
        p = torch.softmax(s, dim=-1).nan_to_num_(0.0)
        del s
        oc = torch.matmul(p.view(B, HK, G * n, m), vs)  # (B, HK, G*n, D)
        out[:, i0:i1] = oc.view(B, HK, G, n, D).permute(0, 3, 1, 2, 4).reshape(B, n, H, D)
        lse[:, :, i0:i1] = lc.reshape(B, H, n)
    return (out, lse) if return_lse else out


def brute_force_attention(q, k, v, lo: int, hi: int):
    """Scalar float64 loops (tiny inputs): o[b,i,h] = sum_j softmax_j(s_ij) v_j over
    lo <= i - j < hi, 0 <= j <= i; returns (o, lse) as float64 tensors."""
    B, T, H, D = q.shape
    HK = k.shape[2]
    G = H // HK
    qd, kd, vd = q.double().tolist(), k.double().tolist(), v.double().tolist()
    o = torch.zeros(B, T, H, D, dtype=torch.float64)
    lse = torch.full((B, H, T), NEG_INF, dtype=torch.float64)
    scale = 1.0 / math.sqrt(D)
    for b in range(B):
        for h in range(H):
            hk = h // G
            for i in range(T):
                js = [j for j in range(0, i + 1) if lo <= i - j < hi]
                if not js:
                    continue
                sc = [sum(qd[b][i][h][d] * kd[b][j][hk][d] for d in range(D)) * scale for j in js]
                mx = max(sc)
                w = [math.exp(x - mx) for x in sc]
                z = sum(w)
                lse[b, h, i] = mx + math.log(z)
                for d in range(D):
                    o[b, i, h, d] = sum(w[t] * vd[b][js[t]][hk][d] for t in range(len(js))) / z
    return o, lse


def lse_merge_reference(o_s, lse_s, o_f, lse_f):
    """lt = logaddexp(ls, lf); o = o_s e^{ls-lt} + o_f e^{lf-lt} (float64).
    o_*: (B, T, H, D), lse_*: (B, H, T). Rows with lse_f = -inf return o_s."""
    ls = lse_s.double()
    lf = lse_f.double()
    lt = torch.logaddexp(ls, lf)
    ws = torch.exp(ls - lt).nan_to_num(0.0).transpose(1, 2).unsqueeze(-1)
    wf = torch.exp(lf - lt).nan_to_num(0.0).transpose(1, 2).unsqueeze(-1)
    return o_s.double() * ws + o_f.double() * wf, lt


# --------------------------------------------------------------------------- emulator
def _f32(x):
    return x.to(torch.float32)


def _fma(a, b, c):
    """fp32 fused multiply-add, via one float64 evaluation (a*b exact in fp64)."""
    return _f32(a.double() * b.double() + c.double())


class _State:
    def __init__(self, bm, d):
        self.acc = torch.zeros(bm, d, dtype=torch.float32)
        self.m = torch.full((bm,), NEG_INF, dtype=torch.float32)
        self.l = torch.zeros(bm, dtype=torch.float32)


def _guard(m, c):
    return torch.where(m == NEG_INF, torch.zeros_like(m), _f32(m * c))


def _full_update(st, s, vblk, c, dt):
    """acc = acc*alpha + bf16(p) @ v; l = l*alpha + sum(p) (fused_dual_attn.py:100-107)."""
    m_new = torch.maximum(st.m, s.max(dim=1).values)
    mc = _guard(m_new, c)
    alpha = torch.exp2(_fma(st.m, c, -mc))
    p = torch.exp2(_fma(s, c, -mc[:, None]))
    pv = p.to(dt).float() @ vblk
    st.acc = _fma(st.acc, alpha[:, None], pv)
    st.l = _fma(st.l, alpha, p.sum(dim=1))
    st.m = m_new
    return mc, p, pv


def _reuse_update(ss, mtc, m_t_new, p, pv, c):
    """Student update from the teacher's P@V by row rescale (:109-116)."""
    m_new = torch.maximum(ss.m, m_t_new)
    msc = _guard(m_new, c)
    alpha = torch.exp2(_fma(ss.m, c, -msc))
    scale = torch.exp2(mtc - msc)
    ss.acc = _fma(ss.acc, alpha[:, None], pv * scale[:, None])
    ss.l = _fma(ss.l, alpha, p.sum(dim=1) * scale)
    ss.m = m_new


def emulate_reference_kernel(q, k, v, window_teacher, window_student, *, block_m: int = 64,
                             block_n: int = 64, row_blocks=None, heads=None):
    """CPU emulation of the reference Triton kernel's numerics; returns
    (o_teacher, o_student) in q.dtype. Used to report the fraction of GPU
    outputs bit-identical to the reference kernel's algorithm (the last bits
    still depend on each device's dot-product reduction order and exp2).

    row_blocks (first rows, multiples of block_m) and heads restrict the
    emulation to those query blocks and heads, as the kernel computes each
    (block, head) independently; the other outputs are left as zeros. This
    samples the 64K shapes, where the whole emulation would take hours."""
    B, T, H, D = q.shape
    HK = k.shape[2]
    G = H // HK
    WT = T if (window_teacher is None or window_teacher < 0) else window_teacher
    WS = window_student
    dt = q.dtype
    c = float(torch.tensor(D ** -0.5, dtype=torch.float32) * torch.tensor(LOG2E, dtype=torch.float32))
    c = torch.tensor(c, dtype=torch.float32)
    BM, BN = block_m, block_n
    ot = torch.zeros(B, T, H, D, dtype=dt)
    os_ = torch.zeros(B, T, H, D, dtype=dt)
    blocks = range(0, T, BM) if row_blocks is None else [int(r) for r in row_blocks]
    assert all(r % BM == 0 and 0 <= r < T for r in blocks), "row blocks start at multiples of block_m"
    for b in range(B):
        for h in (range(H) if heads is None else heads):
            hk = h // G
            kh = torch.zeros(T + BN, D)
            vh = torch.zeros(T + BN, D)
            kh[:T] = k[b, :, hk].float()
            vh[:T] = v[b, :, hk].float()
            qf = q[b, :, h].float()
            for m_start in blocks:
                rows = torch.arange(m_start, m_start + BM)
                qb = torch.zeros(BM, D)
                nval = min(BM, T - m_start)
                qb[:nval] = qf[m_start:m_start + nval]
                st, ss = _State(BM, D), _State(BM, D)
                m_end = m_start + BM - 1
                nb_last = m_end // BN
                nb_diag = m_start // BN
                nb_s_full = max(-((-(m_start + BM - WS)) // BN), 0)
                nb_s_any = max((m_start - WS + 1) // BN, 0)
                nb_t_full = max(-((-(m_start + BM - WT)) // BN), 0)
                nb_t_any = max((m_start - WT + 1) // BN, 0)

                def tile(nb):
                    cols = torch.arange(nb * BN, nb * BN + BN)
                    s = qb @ kh[nb * BN:nb * BN + BN].T
                    return cols, s, vh[nb * BN:nb * BN + BN]

                for nb in range(nb_last, nb_diag - 1, -1):          # A: diagonal
                    cols, s, vb = tile(nb)
                    dist = rows[:, None] - cols[None, :]
                    s = s.masked_fill(~((dist >= 0) & (cols[None, :] < T)), NEG_INF)
                    mtc, p, pv = _full_update(st, s, vb, c, dt)
                    _reuse_update(ss, mtc, st.m, p, pv, c)
                for nb in range(nb_diag - 1, nb_s_full - 1, -1):    # B: shared interior
                    cols, s, vb = tile(nb)
                    mtc, p, pv = _full_update(st, s, vb, c, dt)
                    _reuse_update(ss, mtc, st.m, p, pv, c)
                if WT >= WS + BM + BN:
                    for nb in range(nb_s_full - 1, nb_s_any - 1, -1):  # C
                        cols, s, vb = tile(nb)
                        _full_update(st, s, vb, c, dt)
                        dist = rows[:, None] - cols[None, :]
                        _full_update(ss, s.masked_fill(~(dist < WS), NEG_INF), vb, c, dt)
                    for nb in range(nb_s_any - 1, nb_t_full - 1, -1):  # D
                        _, s, vb = tile(nb)
                        _full_update(st, s, vb, c, dt)
                    for nb in range(nb_t_full - 1, nb_t_any - 1, -1):  # E
                        cols, s, vb = tile(nb)
                        dist = rows[:, None] - cols[None, :]
                        _full_update(st, s.masked_fill(~(dist < WT), NEG_INF), vb, c, dt)
                else:
                    for nb in range(nb_s_full - 1, nb_t_any - 1, -1):  # narrow gap
                        cols, s, vb = tile(nb)
                        dist = rows[:, None] - cols[None, :]
                        _full_update(st, s.masked_fill(~(dist < WT), NEG_INF), vb, c, dt)
                        _full_update(ss, s.masked_fill(~(dist < WS), NEG_INF), vb, c, dt)
                for state, out in ((st, ot), (ss, os_)):
                    inv = _f32(1.0 / state.l.double())
                    o = (state.acc * inv[:, None]).to(dt)
                    out[b, m_start:m_start + nval, h] = o[:nval]
    return ot, os_


# --------------------------------------------------------------------------- reports
def _ordered_bits(x: torch.Tensor) -> torch.Tensor:
    i = x.contiguous().view(torch.int16).to(torch.int32)
    return torch.where(i < 0, -32768 - i, i)


def ulp_report(a: torch.Tensor, ref: torch.Tensor) -> dict:
    """bf16/fp16 distance in units in the last place (profiling/fused_dual_attn.py:275-286):
    bit patterns mapped to a monotone integer scale; percentages of equal,
    <= 1 ulp, <= 2 ulp, and the max distance."""
    d = (_ordered_bits(a.cpu()) - _ordered_bits(ref.cpu())).abs()
    n = d.numel()
    return {
        "bit_equal_pct": (d == 0).sum().item() / n * 100.0,
        "le1ulp_pct": (d <= 1).sum().item() / n * 100.0,
        "le2ulp_pct": (d <= 2).sum().item() / n * 100.0,
        "max_ulp": int(d.max().item()) if n else 0,
    }


def error_stats(actual: torch.Tensor, expected: torch.Tensor) -> tuple[float, float]:
    """(max |diff|, mean |diff|) in fp32, as test_fused_dual_attn.py:113-115."""
    diff = (actual.float().cpu() - expected.float().cpu()).abs()
    return diff.max().item(), diff.mean().item()
