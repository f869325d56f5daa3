"""SwiGLU MLP and the TTT MLP of ipttcdv9 on the GPU (host side of ttt.hip).

    swiglu(gate, up)                      fla's swiglu forward
    swiglu_mlp(x, gate_up_w, down_w)      the plain MLP (swiglu_linear)
    ttt_features(gu_t, gu_s, ...)         the feature pass: both swiglus, both
                                          chunk-local convs, their difference
    ttt_mlp(x, t, weights, ...)           the TTT MLP forward (scanfuse form)

The TTT MLP follows custom_models/ipttcd/modeling_ipttcdv9_lowcopy_scanfuse.py:
36-204 (the implementation bench_prefill.py runs by default), with the
chunk-local conv that profiling/patches.py:411-432 patches in, for the
options the IP-TTCD configs use: fused ttt_proj, dynamic lr, no student
feature normalisation, no normalised proj-diff, no Muon, no weight renorm.
Its GEMMs run on hipBLASLt through torch, one launch per reference matmul
(per chunk where the reference multiplies per chunk); the element-wise
passes between them are the HIP kernels, or torch element-wise ops where
the reference's own rounding (bf16 cumsum, bf16 adds) is what matters.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib

_DT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16,
       torch.float32: _lib.DTYPE_F32}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_gpu(fn: str, **tensors):
    for name, t in tensors.items():
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError(f"{fn}: {name} must be a tensor on a GPU (HIP) device")
        if torch.is_grad_enabled() and t.requires_grad:
            raise RuntimeError(f"{fn} is forward-only: call it under torch.no_grad()")


def _row_stride(t: torch.Tensor, fn: str, name: str) -> int:
    """Element stride between consecutive rows of t seen as (rows, t.shape[-1]):
    the last dim must be contiguous and the leading dims evenly strided (a
    contiguous tensor, or a column slice of one, such as half of a GEMM output)."""
    if t.dim() < 1 or t.stride(-1) != 1:
        raise ValueError(f"{fn}: {name} must have a contiguous last dim")
    if t.dim() == 1 or t.is_contiguous():
        return t.shape[-1]
    st = t.stride(-2)
    expect = st
    for d in range(t.dim() - 2, -1, -1):
        if t.shape[d] != 1 and t.stride(d) != expect:
            raise ValueError(f"{fn}: {name} rows must be evenly strided")
        expect *= t.shape[d]
    return st


def swiglu(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """(g * sigmoid(g)) * u in fp32, rounded (fla/modules/activations.py:412-471).
    gate / up may be row-strided views (e.g. the halves of one GEMM output)."""
    _check_gpu("swiglu", gate=gate, up=up)
    if gate.shape != up.shape or gate.dtype != up.dtype or gate.dtype not in (torch.bfloat16,
                                                                              torch.float16):
        raise ValueError("swiglu: gate and up must share a shape and a bf16/f16 dtype")
    cols = gate.shape[-1]
    g_st, u_st = _row_stride(gate, "swiglu", "gate"), _row_stride(up, "swiglu", "up")
    if out is None:
        out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    rows = gate.numel() // cols if cols else 0
    if rows:
        _lib.check(_lib.lib().ttcd_swiglu_fwd(
            gate.data_ptr(), up.data_ptr(), out.data_ptr(), rows, cols, g_st, u_st,
            _row_stride(out, "swiglu", "out"), _DT[gate.dtype], _stream(gate)))
    return out


def swiglu_mlp(x: torch.Tensor, gate_up_w: torch.Tensor, down_w: torch.Tensor) -> torch.Tensor:
    """fla's swiglu_linear(gate_proj(x), up_proj(x), down_proj.weight)
    (custom_models/ipttcd/modeling_ipttcdv9.py:253-255; activations.py:508-540)
    with gate_proj and up_proj as one GEMM over the stacked (2*I, H) weight."""
    I = gate_up_w.shape[0] // 2
    gu = F.linear(x, gate_up_w)
    z = swiglu(gu[..., :I], gu[..., I:])
    return F.linear(z, down_w)


def ttt_features(gu_t: torch.Tensor, gu_s: torch.Tensor, conv_t: torch.Tensor | None,
                 conv_s: torch.Tensor | None, B: int, nchunk: int, chunk: int):
    """gu_t / gu_s: (B*nchunk*chunk, 2*I) gate|up rows of the teacher / student.
    conv_*: (I, K) (or the module's (I, 1, K)) depthwise causal conv weights or
    None. Returns (z, z_hat, diff): z (rows, I) teacher features, z_hat the
    student's after its conv, diff = conv_t(z) - z_hat for every chunk but the
    last of each batch row, (B*(nchunk-1)*chunk, I)."""
    rows = B * nchunk * chunk
    if gu_t.shape != gu_s.shape or gu_t.dim() != 2 or gu_t.shape[0] != rows:
        raise ValueError(f"ttt_features: gate|up must be ({rows}, 2*I), got {tuple(gu_t.shape)}")
    if gu_t.stride() != gu_s.stride() or gu_t.stride(1) != 1:
        raise ValueError("ttt_features: teacher and student gate|up must share a row stride")
    I = gu_t.shape[1] // 2
    # Every present weight must have the first present weight's kernel size:
    # the kernel reads K taps of each, so a shorter one would be over-read.
    ws = []
    K = None
    for w in (conv_t, conv_s):
        if w is None:
            ws.append(None)
            continue
        w2 = w.reshape(w.shape[0], -1)
        if w2.shape[0] != I:
            raise ValueError(f"ttt_features: conv weight must be ({I}, K)")
        if K is not None and w2.shape[1] != K:
            raise ValueError("ttt_features: both convs must share a kernel size")
        K = w2.shape[1]
        ws.append(w2)
    if K is None:
        K = 1
    if ws[0] is not None and ws[1] is not None and ws[0].dtype != ws[1].dtype:
        raise ValueError("ttt_features: both conv weights must share a dtype")
    _check_gpu("ttt_features", gu_t=gu_t, gu_s=gu_s, conv_t=conv_t, conv_s=conv_s)
    ws = [w.contiguous() if w is not None else None for w in ws]
    wdt = next((w.dtype for w in ws if w is not None), torch.float32)
    dev, dt = gu_t.device, gu_t.dtype
    z = torch.empty(rows, I, dtype=dt, device=dev)
    z_hat = torch.empty(rows, I, dtype=dt, device=dev)
    diff = torch.empty(B * (nchunk - 1) * chunk, I, dtype=dt, device=dev)
    _lib.check(_lib.lib().ttcd_ttt_features_fwd(
        gu_t.data_ptr(), gu_s.data_ptr(), gu_t.stride(0),
        ws[0].data_ptr() if ws[0] is not None else None,
        ws[1].data_ptr() if ws[1] is not None else None, _DT[wdt], K, z.data_ptr(),
        z_hat.data_ptr(), diff.data_ptr() if nchunk > 1 else None, B, nchunk, chunk, I,
        _DT[dt], _stream(gu_t)))
    return z, z_hat, diff


def _stack_rows(x: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
    """(2*rows, H) view of [x; t] when they are adjacent halves of one buffer,
    else a copy."""
    H = x.shape[-1]
    n = x.numel()
    if (x.is_contiguous() and t.is_contiguous()
            and t.data_ptr() == x.data_ptr() + n * x.element_size()
            and x.untyped_storage().data_ptr() == t.untyped_storage().data_ptr()):
        return torch.as_strided(x, (2 * (n // H), H), (H, 1))
    return torch.cat([x.reshape(-1, H), t.reshape(-1, H)], dim=0)


def proj_beta_t(pd: torch.Tensor, beta: torch.Tensor | None, B: int, nupd: int,
                chunk: int) -> torch.Tensor:
    """pd (B*nupd*chunk, H) -> (B*nupd, H, chunk) = per chunk (pd * beta)^T,
    one rounding per element (scanfuse.py:126-127). beta: (B, >= nupd, chunk)
    per-token learning rates or None."""
    H = pd.shape[1]
    if pd.dim() != 2 or pd.stride(1) != 1 or pd.shape[0] != B * nupd * chunk:
        raise ValueError("proj_beta_t: pd must be (B*nupd*chunk, H) with a contiguous row")
    bsb = 0
    if beta is not None:
        if beta.dim() != 3 or beta.shape[0] != B or beta.shape[1] < nupd or beta.shape[2] != chunk \
                or not beta.is_contiguous() or beta.dtype != pd.dtype:
            raise ValueError("proj_beta_t: beta must be contiguous (B, >= nupd, chunk) of pd's dtype")
        bsb = beta.stride(0)
    _check_gpu("proj_beta_t", pd=pd, beta=beta)
    out = torch.empty(B * nupd, H, chunk, dtype=pd.dtype, device=pd.device)
    _lib.check(_lib.lib().ttcd_ttt_proj_beta_t_fwd(
        pd.data_ptr(), pd.stride(0), beta.data_ptr() if beta is not None else None, bsb,
        out.data_ptr(), B, nupd, chunk, H, _DT[pd.dtype], _stream(pd)))
    return out


def scan_steps(dw: torch.Tensor | None, w_cur: torch.Tensor, lr: float, nsteps: int,
               want_next: bool):
    """One update group: dw (nupd, H, I) chunk updates, w_cur (H, I). Returns
    (steps_t, w_next): steps_t (nsteps, I, H) with step 0 = w_cur^T and step s
    = (w_cur + lr * cumsum(dw)[s-1])^T, every step rounded as torch's bf16 ops
    round it (scanfuse.py:157-170); w_next = w_cur + lr * cumsum(dw)[-1] or
    None."""
    H, I = w_cur.shape
    nupd = 0 if dw is None else dw.shape[0]
    if dw is not None and (dw.shape[1:] != (H, I) or not dw.is_contiguous()
                           or dw.dtype != w_cur.dtype):
        raise ValueError("scan_steps: dw must be contiguous (nupd, H, I) of w_cur's dtype")
    if not w_cur.is_contiguous():
        raise ValueError("scan_steps: w_cur must be contiguous")
    _check_gpu("scan_steps", dw=dw, w_cur=w_cur)
    dt = w_cur.dtype
    lr_q = float(torch.tensor(lr, dtype=dt).item())   # the learning rate as the dtype stores it
    steps = torch.empty(nsteps, I, H, dtype=dt, device=w_cur.device)
    w_next = torch.empty(H, I, dtype=dt, device=w_cur.device) if want_next else None
    _lib.check(_lib.lib().ttcd_ttt_scan_fwd(
        dw.data_ptr() if dw is not None else None, w_cur.data_ptr(), lr_q, steps.data_ptr(),
        w_next.data_ptr() if w_next is not None else None, nupd, nsteps, H, I, _DT[dt],
        _stream(w_cur)))
    return steps, w_next


def _scan_kernel(pd, beta, z4, zh4, W_base, out, *, lr, update_every):
    """The group loop of scanfuse.py:121-172 on the update kernels and
    batched GEMMs. pd (B*(nchunk-1)*C, H); z4 / zh4 (B, nchunk, C, I);
    out (B, nchunk, C, H)."""
    B, nchunk, C, I = z4.shape
    K = nchunk - 1
    pdt = proj_beta_t(pd, beta, B, K, C)               # (B*K, H, C)
    G = max(1, min(nchunk, update_every))
    W_base = W_base.contiguous()
    for b in range(B):
        # every chunk's update at once: (K, H, C) @ (K, C, I) -> (K, H, I)
        dW = torch.bmm(pdt[b * K:(b + 1) * K], zh4[b, :K])
        W_cur = W_base
        for gs in range(0, nchunk, G):
            ge = min(gs + G, nchunk)
            upd_end = min(ge, K)
            last = ge >= nchunk
            steps, W_next = scan_steps(dW[gs:upd_end] if upd_end > gs else None, W_cur, lr,
                                       ge - gs, want_next=not last and upd_end > gs)
            # the group's outputs: (Kg, C, I) @ (Kg, I, H) -> (Kg, C, H)
            torch.bmm(z4[b, gs:ge], steps, out=out[b, gs:ge])
            if W_next is not None:
                W_cur = W_next


class TttMlpWeights:
    """The TTT MLP's parameters, named after the reference module's
    (custom_models/ipttcd/modeling_ipttcdv9.py:87-182)."""

    def __init__(self, gate_up: torch.Tensor, down: torch.Tensor, ttt_proj: torch.Tensor | None,
                 conv_t: torch.Tensor | None, conv_s: torch.Tensor | None,
                 b_proj: torch.Tensor | None):
        self.gate_up, self.down, self.ttt_proj = gate_up, down, ttt_proj
        self.conv_t, self.conv_s, self.b_proj = conv_t, conv_s, b_proj


def stock_conv(v: torch.Tensor, cw: torch.Tensor) -> torch.Tensor:
    """The reference's unpatched chunk-local conv (IPTTCDMLP._apply_ttt_conv,
    modeling_ipttcdv9.py:203-211): (b, t, c, d) -> ((b t), d, c), left pad
    K-1, torch's depthwise conv1d (MIOpen), back. The A/B baseline of the conv
    kernel; its accumulation order is MIOpen's, not fixed."""
    b, t, c, d = v.shape
    K = cw.shape[-1]
    xf = F.pad(v.permute(0, 1, 3, 2).reshape(b * t, d, c), (K - 1, 0))
    y = F.conv1d(xf, cw.reshape(d, 1, K), groups=d)
    return y.reshape(b, t, d, c).permute(0, 1, 3, 2).contiguous()


def ttt_mlp(x: torch.Tensor, t: torch.Tensor, w: TttMlpWeights, *, chunk: int, lr: float,
            update_every: int, fused: bool = True, conv: str = "kernel",
            scan: str = "kernel") -> torch.Tensor:
    """The TTT MLP forward for a prefill: x the teacher hidden states after
    mlp_norm, t the student's (B, L, H). Returns the MLP output (B, L, H).

    Per chunk c of C tokens (the scanfuse loop, scanfuse.py:100-172, in groups
    of min(nchunk, update_every) chunks):
        diff_c  = conv_t(z)_c - z_hat_c
        pd_c    = (diff_c @ (W_down^T @ P)) * beta_c     P = ttt_proj.weight
        dW_c    = pd_c^T @ z_hat_c
        W_c     = W_cur + lr * cumsum_group(dW)[c - 1]    (W_cur at the group start)
        y_c     = z_c @ W_c^T
    with W_cur = W_down for the first group and advanced by the group's last
    cumsum at its end. `fused=False` runs the feature pass as separate launches
    (swiglu, conv, subtraction) for A/B measurement, with the conv kernel
    (conv="kernel": identical results) or the reference's unpatched torch
    conv (conv="stock"). scan="kernel" runs the update scan as the
    reference's group loop does it but batched: one GEMM for pd, one kernel
    for pd * beta (transposed per chunk), one batched GEMM for every chunk's
    dW, and per group one scan kernel (bf16 running sum, lr * sum, W_cur + cs
    for every chunk, transposed) and one batched GEMM for the group's outputs;
    scan="torch" runs the reference's per-chunk torch ops (the same roundings;
    the GEMMs' accumulation order may differ)."""
    from .conv import causal_dwconv_x

    B, L, H = x.shape
    C = chunk
    I = w.gate_up.shape[0] // 2
    nchunk = (L + C - 1) // C
    pad = nchunk * C - L
    dt, dev = x.dtype, x.device
    if pad:
        x = F.pad(x, (0, 0, 0, pad))
        t = F.pad(t, (0, 0, 0, pad))
    rows = B * nchunk * C
    gu = F.linear(_stack_rows(x, t), w.gate_up)  # one GEMM over teacher and student rows
    gu_t, gu_s = gu[:rows], gu[rows:]
    if conv not in ("kernel", "stock"):
        raise ValueError(f"ttt_mlp: conv must be 'kernel' or 'stock', got {conv!r}")
    if scan not in ("kernel", "torch"):
        raise ValueError(f"ttt_mlp: scan must be 'kernel' or 'torch', got {scan!r}")
    if fused and conv == "kernel":
        z, z_hat, diff = ttt_features(gu_t, gu_s, w.conv_t, w.conv_s, B, nchunk, C)
    else:
        z = swiglu(gu_t[:, :I], gu_t[:, I:])
        z_raw = swiglu(gu_s[:, :I], gu_s[:, I:])

        def apply_conv(v, cw):
            if cw is None:
                return v
            if conv == "stock":
                return stock_conv(v.view(B, nchunk, C, I), cw).view(rows, I)
            return causal_dwconv_x(v.view(B * nchunk, C, I), cw.reshape(I, -1)).view(rows, I)

        z_tgt = apply_conv(z, w.conv_t)
        z_hat = apply_conv(z_raw, w.conv_s)
        keep = torch.arange(nchunk, device=dev) < nchunk - 1
        diff = (z_tgt.view(B, nchunk, C, I)[:, keep] - z_hat.view(B, nchunk, C, I)[:, keep])
        diff = diff.reshape(-1, I)

    W_base = w.down                                   # (H, I)
    z4 = z.view(B, nchunk, C, I)
    out = torch.empty(B, nchunk, C, H, dtype=dt, device=dev)
    if nchunk > 1:
        beta = None
        if w.b_proj is not None:
            # (t_padded @ b_proj).sigmoid(), bf16 (scanfuse.py:72-74)
            beta = torch.matmul(t.view(B, nchunk, C, H), w.b_proj).sigmoid()
        W_upd_t = W_base.t()
        if w.ttt_proj is not None:
            W_upd_t = torch.matmul(W_base.t(), w.ttt_proj)  # (I, H), scanfuse.py:95-96
        pd = torch.mm(diff, W_upd_t)                  # (B*(nchunk-1)*C, H)
        if scan == "kernel":
            _scan_kernel(pd, beta, z4, z_hat.view(B, nchunk, C, I), W_base, out, lr=lr,
                         update_every=update_every)
            return out.view(B, nchunk * C, H)[:, :L]
        pd = pd.view(B, nchunk - 1, C, H)
        if beta is not None:
            pd = pd * beta[:, :nchunk - 1, :, None]
        zh4 = z_hat.view(B, nchunk, C, I)
        dW = torch.empty(B, nchunk - 1, H, I, dtype=dt, device=dev)
        for b in range(B):
            for c in range(nchunk - 1):
                torch.mm(pd[b, c].t(), zh4[b, c], out=dW[b, c])
        lr_t = torch.tensor(lr, dtype=dt, device=dev)
        G = max(1, min(nchunk, update_every))
        for b in range(B):
            W_cur = W_base
            for gs in range(0, nchunk, G):
                ge = min(gs + G, nchunk)
                upd_end = min(ge, nchunk - 1)
                cs = lr_t * torch.cumsum(dW[b, gs:upd_end], dim=0) if upd_end > gs else None
                for ci in range(gs, ge):
                    if ci == gs or cs is None:
                        W_step = W_cur
                    else:
                        W_step = W_cur + cs[min(ci - gs - 1, upd_end - gs - 1)]
                    torch.mm(z4[b, ci], W_step.t(), out=out[b, ci])
                if cs is not None:
                    W_cur = W_cur + cs[-1]
    else:
        for b in range(B):
            torch.mm(z4[b, 0], W_base.t(), out=out[b, 0])
    return out.view(B, nchunk * C, H)[:, :L]
