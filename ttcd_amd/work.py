"""Algorithmic work per launch: the figures throughput and roofline fractions
are computed from (FLOPs for the MFMA-bound attention, HBM bytes for the
bandwidth-bound passes). Counts only what the algorithm must do, never what a
kernel happens to do (re-reads, masked tiles, the student band's reuse).
"""
from __future__ import annotations


def band_pairs(T: int, lo: int, hi: int) -> int:
    """#(i, j) with 0 <= j <= i < T and lo <= i - j < hi."""
    hi = min(hi, T)
    if hi <= lo:
        return 0
    n = hi - lo
    return n * T - (lo + hi - 1) * n // 2


def window_pairs(T: int, W: int | None) -> int:
    """P(T, W) = W(W+1)/2 + (T-W)W for W <= T, else T(T+1)/2 (full causal)."""
    if W is None or W < 0 or W >= T:
        return T * (T + 1) // 2
    return W * (W + 1) // 2 + (T - W) * W


def attn_flops(B: int, H: int, D: int, T: int, W: int | None) -> int:
    """QK^T and PV over the window: 4 * D FLOPs per visible (query, key) pair.
    For the dual-window kernel W is the teacher window (the student band is a
    subset, recovered by reuse, and not counted again)."""
    return 4 * B * H * D * window_pairs(T, W)


def conv_bytes(N: int, C: int, D: int, K: int, elem: int = 2, w_elem: int = 2) -> int:
    """Chunked depthwise conv: read x once, write y once, read the weights."""
    return 2 * N * C * D * elem + D * K * w_elem


def prologue_bytes(B: int, T: int, Hq: int, Hkv: int, D: int, elem: int = 2) -> int:
    """q/k RMSNorm + rotary in one launch: q and k read once and written once,
    plus the cos/sin rows (T x D elements, shared by every head)."""
    return 2 * B * T * (Hq + Hkv) * D * elem + 2 * T * (D // 2) * elem


def epilogue_bytes(rows: int, hidden: int, elem: int = 2, w_elem: int = 2) -> int:
    """Dual residual RMSNorm: three (rows, hidden) reads (attn_t, attn_s,
    residual), three writes (hidden_states, residual_out, student_output),
    the weight once."""
    return 6 * rows * hidden * elem + hidden * w_elem


def merge_bytes(B: int, T: int, H: int, D: int, row_start: int, elem: int = 2) -> int:
    """LSE merge: rows >= row_start read o_s, o_f and both LSEs and write o_t;
    rows below copy o_s."""
    tail = max(T - row_start, 0)
    return B * H * (tail * (3 * D * elem + 8) + (T - tail) * 2 * D * elem)
