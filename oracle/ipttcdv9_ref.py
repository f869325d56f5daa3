"""CPU oracle for the ipttcdv9 prefill (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py may use this module, as
the checker.

A plain-torch restatement of the reference's prefill on the CPU, op by op,
computing each op in fp32 (float64 where stated) from the stored inputs and
rounding its result to the model dtype where the reference stores it:

  swiglu_ref            fla swiglu_fwd_kernel (fla/modules/activations.py:
                        412-426): (g * sigmoid(g)) * u in fp32.
  ttt_mlp_scan_ref      the TTT MLP forward as the reference's group loop
                        (custom_models/ipttcd/modeling_ipttcdv9_lowcopy_
                        scanfuse.py:36-204): per group of chunks, cumsum of
                        the chunk updates, W for chunk c = W_cur + cs[c-1];
                        the bf16 cumsum accumulates with a rounding per step,
                        as torch's GPU scan over a bf16 tensor does.
  ttt_mlp_token_f64     the same map written per token in float64, with no
                        chunk GEMMs: y_t = z_t (W_down + lr sum over earlier
                        chunks' tokens of beta_s pd_s (x) zhat_s)^T, the
                        cumsum form of profiling/patches.py:487-506.
  prefill_ref           IPTTCDForCausalLM prefill logits (modeling_ipttcdv9.py:
                        577-880, 999-1128, 1194-1241; fla/layers/attn.py:
                        170-270): RMSNorm, q|k|v projections, q/k RMSNorm +
                        rotary, windowed causal attention (attn_ref.
                        band_reference), o_proj, residual RMSNorm, SwiGLU MLP
                        or the TTT MLP, final norm, LM head; optionally one
                        chunk of a prompt prefilled over a K/V cache
                        (new_cache_ref).

Pins (tests/test_ipttcdv9.py): ttt_mlp_scan_ref in float64 == ttt_mlp_token_f64
(two formulations: chunk GEMMs + grouped cumsum vs per-token outer products),
for one and several groups and a ragged last chunk; a planted off-by-one
(chunk c using its own update) fails it; lr = 0 and teacher == student
features reduce to the plain MLP z @ W_down^T; swiglu_ref against
x * sigmoid(x) * y in float64 within one rounding; prefill_ref with no TTT
layers and window >= T equals a dense causal transformer written with
dense_reference; a prompt prefilled in chunks over the cache, with no TTT
layers (whose MLP restarts per chunk), gives the one-shot prefill's logits,
also when the cache has been trimmed to the window, and a planted mistake
(a rotary offset that does not continue) does not; the components it
composes are pinned in their own test files (attention, rotary, RMSNorm,
conv).
"""
from __future__ import annotations

import math

import torch

from . import attn_ref, conv_ref, epilogue_ref, prologue_ref


def _mm(a: torch.Tensor, b: torch.Tensor, dt) -> torch.Tensor:
    """a @ b of stored values, fp32 accumulation, result stored as dt."""
    return (a.float() @ b.float()).to(dt)


def swiglu_ref(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    gf, uf = g.float(), u.float()
    s = 1.0 / (1.0 + torch.exp(-gf))
    return ((gf * s) * uf).to(g.dtype)


def cumsum_stepwise(x: torch.Tensor, dim: int = 0) -> torch.Tensor:
    """Inclusive scan with the running sum stored in x's dtype after every
    step (torch's GPU scan of a bf16 tensor)."""
    xs = x.movedim(dim, 0)
    out = torch.empty_like(xs)
    acc = torch.zeros_like(xs[0])
    for i in range(xs.shape[0]):
        acc = (acc.float() + xs[i].float()).to(x.dtype)
        out[i] = acc
    return out.movedim(0, dim)


def conv_chunks(z: torch.Tensor, w: torch.Tensor | None) -> torch.Tensor:
    """z (B, nchunk, C, I); w (I, 1, K) or None -> chunk-local causal conv,
    fp32 taps in order, rounded (profiling/fused_conv.py:39-48)."""
    if w is None:
        return z
    B, N, C, I = z.shape
    w2 = w.reshape(I, -1)
    if z.dtype in (torch.bfloat16, torch.float16) and w2.dtype in (torch.bfloat16, torch.float16):
        y = conv_ref.dwconv_numpy(z.reshape(B * N, C, I), w2)
        return y.reshape(B, N, C, I).to(z.dtype)
    # wider dtypes: the same taps in order, in float64
    K = w2.shape[1]
    x = torch.nn.functional.pad(z.double(), (0, 0, K - 1, 0))
    y = torch.zeros(B, N, C, I, dtype=torch.float64)
    for j in range(K):
        y = y + x[:, :, j:j + C] * w2[:, j].double()
    return y.to(z.dtype)


def ttt_features_ref(gu_t, gu_s, conv_t, conv_s, B, nchunk, C):
    """(z, z_hat, diff) as the reference's launches store them; gu_* are
    (B*nchunk*C, 2I) gate|up rows."""
    I = gu_t.shape[1] // 2
    z = swiglu_ref(gu_t[:, :I], gu_t[:, I:]).reshape(B, nchunk, C, I)
    zr = swiglu_ref(gu_s[:, :I], gu_s[:, I:]).reshape(B, nchunk, C, I)
    z_tgt = conv_chunks(z, conv_t)
    z_hat = conv_chunks(zr, conv_s)
    diff = (z_tgt[:, :nchunk - 1].float() - z_hat[:, :nchunk - 1].float()).to(z.dtype)
    return z.reshape(-1, I), z_hat.reshape(-1, I), diff.reshape(-1, I)


def ttt_mlp_scan_ref(z, z_hat, diff, t_pad, w_down, ttt_proj, b_proj, *, lr, update_every,
                     B, nchunk, C, dt=None):
    """The group loop of scanfuse.py:100-172 on stored tensors.
    z, z_hat: (B*nchunk*C, I); diff: (B*(nchunk-1)*C, I); t_pad: (B, nchunk*C, H)
    student hidden (zero-padded); w_down: (H, I). Returns (B, nchunk*C, H).
    dt: storage dtype (default z's; float64 runs the same map unrounded)."""
    dt = dt or z.dtype
    I = z.shape[1]
    H = w_down.shape[0]
    z4 = z.reshape(B, nchunk, C, I).to(dt)
    zh4 = z_hat.reshape(B, nchunk, C, I).to(dt)
    W_base = w_down.to(dt)
    out = torch.empty(B, nchunk, C, H, dtype=dt)
    if nchunk == 1:
        for b in range(B):
            out[b, 0] = _mm(z4[b, 0], W_base.t(), dt) if dt != torch.float64 else z4[b, 0] @ W_base.t()
        return out.reshape(B, nchunk * C, H)
    mm = (lambda a, b_: a @ b_) if dt == torch.float64 else (lambda a, b_: _mm(a, b_, dt))
    beta = None
    if b_proj is not None:
        logits = mm(t_pad.to(dt).reshape(B, nchunk, C, H), b_proj.to(dt)[:, None])[..., 0]
        beta = torch.sigmoid(logits.double()).to(dt) if dt != torch.float64 else torch.sigmoid(logits)
    W_upd_t = W_base.t()
    if ttt_proj is not None:
        W_upd_t = mm(W_base.t(), ttt_proj.to(dt))
    pd = mm(diff.reshape(-1, I).to(dt), W_upd_t).reshape(B, nchunk - 1, C, H)
    if beta is not None:
        pd = (pd.double() * beta[:, :nchunk - 1, :, None].double()).to(dt)
    dW = torch.empty(B, nchunk - 1, H, I, dtype=dt)
    for b in range(B):
        for c in range(nchunk - 1):
            dW[b, c] = mm(pd[b, c].t(), zh4[b, c])
    lr_s = torch.tensor(lr, dtype=dt)
    G = max(1, min(nchunk, update_every))
    for b in range(B):
        W_cur = W_base
        for gs in range(0, nchunk, G):
            ge = min(gs + G, nchunk)
            upd_end = min(ge, nchunk - 1)
            cs = None
            if upd_end > gs:
                csum = (torch.cumsum(dW[b, gs:upd_end], 0) if dt == torch.float64
                        else cumsum_stepwise(dW[b, gs:upd_end], 0))
                cs = (lr_s.double() * csum.double()).to(dt)
            for ci in range(gs, ge):
                if ci == gs or cs is None:
                    W_step = W_cur
                else:
                    W_step = (W_cur.double() + cs[min(ci - gs - 1, upd_end - gs - 1)].double()).to(dt)
                out[b, ci] = mm(z4[b, ci], W_step.t())
            if cs is not None:
                W_cur = (W_cur.double() + cs[-1].double()).to(dt)
    return out.reshape(B, nchunk * C, H)


def ttt_mlp_token_f64(z, z_hat, diff, t_pad, w_down, ttt_proj, b_proj, *, lr, B, nchunk, C):
    """Per-token float64 form: for token s of chunk c(s) < nchunk-1,
    u_s = beta_s * (diff_s @ W_down^T @ P) and the update U = sum u_s (x) zhat_s;
    token t uses W_down + lr * sum of updates of all chunks before c(t)."""
    I = z.shape[1]
    H = w_down.shape[0]
    zd = z.double().reshape(B, nchunk * C, I)
    zhd = z_hat.double().reshape(B, nchunk * C, I)
    dd = diff.double().reshape(B, (nchunk - 1) * C, I)
    Wd = w_down.double()
    Wu = Wd.t() @ (ttt_proj.double() if ttt_proj is not None else torch.eye(H, dtype=torch.float64))
    out = torch.empty(B, nchunk * C, H, dtype=torch.float64)
    for b in range(B):
        beta = (torch.sigmoid(t_pad[b].double() @ b_proj.double()) if b_proj is not None
                else torch.ones(nchunk * C, dtype=torch.float64))
        acc = Wd.clone()
        for c in range(nchunk):
            rows = slice(c * C, (c + 1) * C)
            out[b, rows] = zd[b, rows] @ acc.t()
            if c < nchunk - 1:
                upd = torch.zeros(H, I, dtype=torch.float64)
                for s in range(c * C, (c + 1) * C):
                    u = beta[s] * (dd[b, s] @ Wu)
                    upd += torch.outer(u, zhd[b, s])
                acc = acc + lr * upd
    return out


def _rope(x, cos, sin):
    return prologue_ref.rope_ref(x, cos, sin, 0)


def _positions(T: int, cu_seqlens) -> torch.Tensor:
    """Rotary positions: 0..T-1, or restarting at every packed sequence
    (fla's rotary with cu_seqlens)."""
    if cu_seqlens is None:
        return torch.arange(T)
    pos = torch.empty(T, dtype=torch.long)
    cu = [int(x) for x in cu_seqlens]
    for a, b in zip(cu[:-1], cu[1:]):
        pos[a:b] = torch.arange(b - a)
    return pos


def output_gate_ref(c: dict, w: dict, p: str, x, o, dt):
    """fla Attention's output gate (fla/layers/attn.py:149-167, 284-292) on
    o (B, T, H, D) with x the attn_norm output: g = x @ g_proj^T; with
    gate_fn 'swish' and fuse_norm, FusedRMSNormGated: rmsnorm(o) * w * g *
    sigmoid(g) in fp32, one rounding (fla/modules/fused_norm_gate.py:91-97);
    otherwise g_norm (RMSNorm over D, stored) times gate_fn(g) (stored), a
    rounded product. Returns (B, T, H*D)."""
    B, T, Hh, D = o.shape
    g = _mm(x, w[p + "attn.g_proj.weight"].t(), dt).view(B, T, Hh, D)
    eps = c["norm_eps"]
    if c["gate_fn"] == "swish" and c["fuse_norm"]:
        of = o.double()
        y = of * torch.rsqrt(of.pow(2).mean(-1, keepdim=True) + eps)
        y = y * w[p + "attn.g_norm_swish_gate.weight"].double()
        gd = g.double()
        y = y * gd * torch.sigmoid(gd)
        return y.to(dt).reshape(B, T, -1)
    on = prologue_ref.rms_norm_ref(o, w[p + "attn.g_norm.weight"], eps)
    gd = g.double()
    act = torch.sigmoid(gd) if c["gate_fn"] == "sigmoid" else gd * torch.sigmoid(gd)
    return (on.double() * act.to(dt).double()).to(dt).reshape(B, T, -1)


def new_cache_ref() -> dict:
    """An empty K/V cache for prefill_ref's chunked prefill: the tokens seen and,
    per layer, the rotated keys and the values kept for the next chunk."""
    return {"seen": 0, "kv": {}}


def _cached_band(q, k_all, v_all, W):
    """Attention of the last Tq positions of a Tk-token sequence (bottom-right
    aligned, window W): band_reference over the full length with the queries
    placed at the end (earlier rows zero and not evaluated)."""
    B, Tq, H, D = q.shape
    Tk = k_all.shape[1]
    qpad = torch.zeros(B, Tk, H, D, dtype=q.dtype)
    qpad[:, Tk - Tq:] = q
    return attn_ref.band_reference(qpad, k_all, v_all, 0, W, rows=torch.arange(Tk - Tq, Tk))


def prefill_ref(cfg: dict, w: dict, input_ids: torch.Tensor, logits_to_keep: int = 1,
                dt=torch.bfloat16, attention_mask=None, cu_seqlens=None,
                cache: dict | None = None) -> torch.Tensor:
    """Logits (B, logits_to_keep, V) of the reference prefill on the CPU.
    cfg: a resolved config (ttcd_amd.ipttcdv9.resolve_config); w: the
    parameters under the reference's state-dict names (CPU tensors).

    attention_mask (B, T) 0/1 padding mask, cu_seqlens packed sequences
    (B = 1): the reference's fallback path (modeling_ipttcdv9.py:562-574,
    794-850). Every layer's attention (fla Attention, fla/layers/attn.py:
    226-262) attends within each row's unpadded tokens or within each packed
    sequence, with rotary positions restarting per packed sequence (not
    shifted for padding: a prefill has no cache). The TTT student is
    flash_attn_func on the whole padded / packed rows (:825-827), and the TTT
    MLP runs on them as they are. Padded rows attend nowhere: o = 0.

    cache (new_cache_ref(), then the same dict for every later chunk): a
    prefill in chunks over a K/V cache. Rotary positions continue from
    cache["seen"]; every layer's attention (teacher window, and the student
    window on TTT layers) runs over the kept keys of the earlier chunks
    followed by the chunk's own, the queries at the end (the flash_attn_func
    calls on the cached k / v of modeling_ipttcdv9.py:741-751, 771-787 and
    fla/layers/attn.py:215-226); each layer then keeps the last window_size
    of them (every key with no window), enough that the next chunk's first
    query sees its whole window; the TTT MLP sees the chunk alone."""
    c = cfg
    B, T = input_ids.shape
    H, I, D = c["hidden_size"], c["intermediate_size"], c["head_dim"]
    Hq, Hkv = c["num_heads"], c["num_kv_heads"]
    eps = c["norm_eps"]
    off = 0 if cache is None else cache["seen"]
    rows_tab = max(off + T, c["max_position_embeddings"] or 0)
    inv = prologue_ref.inv_freq_ref(D, c["rope_theta"])
    cos, sin = prologue_ref.tables_ref(inv, rows_tab, dt)
    pos = _positions(T, cu_seqlens) + off
    cos, sin = cos[pos], sin[pos]
    Wt = c["window_size"] if c["window_size"] is not None else off + T
    Ws = c["ttt_visible_chunks"] * c["ttt_chunk"]
    if attention_mask is not None and bool(attention_mask.all()):
        attention_mask = None

    def norm(x, wt):
        return prologue_ref.rms_norm_ref(x, wt, eps)

    def attn(q, k, v, W):
        if k.shape[1] > q.shape[1]:
            return _cached_band(q, k, v, W).to(dt)
        return attn_ref.band_reference(q, k, v, 0, W).to(dt)

    def teacher_attn(q, k, v):
        if attention_mask is not None:
            o = torch.zeros_like(q)
            for b in range(B):
                idx = attention_mask[b].nonzero().flatten()
                if idx.numel():
                    o[b, idx] = attn(q[b:b + 1, idx], k[b:b + 1, idx], v[b:b + 1, idx], Wt)[0]
            return o
        if cu_seqlens is not None:
            o = torch.zeros_like(q)
            cu = [int(x) for x in cu_seqlens]
            for a, e in zip(cu[:-1], cu[1:]):
                if e > a:
                    o[:, a:e] = attn(q[:, a:e], k[:, a:e], v[:, a:e], Wt)
            return o
        return attn(q, k, v, Wt)

    def gated(p, x, o):
        if c["use_output_gate"]:
            return output_gate_ref(c, w, p, x, o, dt)
        return o.reshape(B, T, -1)

    h = w["model.embeddings.weight"][input_ids].to(dt)
    for i in range(c["num_hidden_layers"]):
        p = f"model.layers.{i}."
        residual = h
        x = norm(h, w[p + "attn_norm.weight"])
        q = _mm(x, w[p + "attn.q_proj.weight"].t(), dt).view(B, T, Hq, D)
        k = _mm(x, w[p + "attn.k_proj.weight"].t(), dt).view(B, T, Hkv, D)
        v = _mm(x, w[p + "attn.v_proj.weight"].t(), dt).view(B, T, Hkv, D)
        if c["qk_norm"]:
            q = prologue_ref.rms_norm_ref(q, w[p + "attn.q_norm.weight"], 1e-5)
            k = prologue_ref.rms_norm_ref(k, w[p + "attn.k_norm.weight"], 1e-5)
        q, k = _rope(q, cos, sin), _rope(k, cos, sin)
        if cache is not None:
            old = cache["kv"].get(i)
            if old is not None:
                k, v = torch.cat([old[0], k], 1), torch.cat([old[1], v], 1)
            n = k.shape[1] if c["window_size"] is None else min(c["window_size"], k.shape[1])
            cache["kv"][i] = (k[:, k.shape[1] - n:], v[:, v.shape[1] - n:])
        o_w = w[p + "attn.o_proj.weight"]
        ttt = i in c["ttt_layers"] and T >= c["ttt_chunk"]
        a_t = _mm(gated(p, x, teacher_attn(q, k, v)), o_w.t(), dt)
        if ttt:
            a_s = _mm(gated(p, x, attn(q, k, v, Ws)), o_w.t(), dt)
            x, residual, s = epilogue_ref.dual_residual_rms_norm_ref(
                a_t, a_s, residual, w[p + "mlp_norm.weight"], eps)
            y = ttt_mlp_ref(c, w, p, x, s, dt)
        else:
            x, residual = epilogue_ref.residual_rms_norm_ref(a_t, residual,
                                                             w[p + "mlp_norm.weight"], eps)
            gate = _mm(x, w[p + "mlp.gate_proj.weight"].t(), dt)
            up = _mm(x, w[p + "mlp.up_proj.weight"].t(), dt)
            y = _mm(swiglu_ref(gate, up), w[p + "mlp.down_proj.weight"].t(), dt)
        h = (residual.float() + y.float()).to(dt)
    if cache is not None:
        cache["seen"] += T
    keep = h[:, -logits_to_keep:] if logits_to_keep > 0 else h
    x = norm(keep, w["model.norm.weight"])
    return _mm(x, w["lm_head.weight"].t(), dt)


def ttt_mlp_ref(c, w, p, x, t, dt):
    """The TTT MLP of layer prefix p on stored x (teacher) and t (student)."""
    B, L, H = x.shape
    C = c["ttt_chunk"]
    nchunk = math.ceil(L / C)
    pad = nchunk * C - L
    if pad:
        x = torch.nn.functional.pad(x, (0, 0, 0, pad))
        t = torch.nn.functional.pad(t, (0, 0, 0, pad))
    gu_w = torch.cat([w[p + "mlp.gate_proj.weight"], w[p + "mlp.up_proj.weight"]], 0)
    gu_t = _mm(x.reshape(-1, H), gu_w.t(), dt)
    gu_s = _mm(t.reshape(-1, H), gu_w.t(), dt)
    z, z_hat, diff = ttt_features_ref(gu_t, gu_s, w.get(p + "mlp.ttt_teacher_conv.weight"),
                                      w.get(p + "mlp.ttt_student_conv.weight"), B, nchunk, C)
    out = ttt_mlp_scan_ref(z, z_hat, diff, t, w[p + "mlp.down_proj.weight"],
                           w.get(p + "mlp.ttt_proj.weight"), w.get(p + "mlp.b_proj"),
                           lr=c["ttt_lr"], update_every=c["ttt_update_every"], B=B,
                           nchunk=nchunk, C=C, dt=dt)
    return out[:, :L]
