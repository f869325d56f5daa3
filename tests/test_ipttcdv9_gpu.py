"""ipttcdv9 prefill on the GPU: the new kernels (RMSNorm, SwiGLU, the TTT
feature pass) through the C ABI against the CPU oracle, the TTT MLP against
the oracle's group loop, and the whole model's logits against the oracle's
prefill on a small config."""
from __future__ import annotations

import pytest
import torch

from oracle import attn_ref, epilogue_ref, ipttcdv9_ref as R, prologue_ref
from ttcd_amd import epilogue, ipttcdv9 as M, ttt

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rand(*shape, seed=0, scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _ulp_ok(got, want, pct=99.0, max_ulp=1):
    rep = attn_ref.ulp_report(got.cpu(), want.cpu())
    assert rep["max_ulp"] <= max_ulp and rep["bit_equal_pct"] > pct, rep


# ------------------------------------------------------------------ kernels


@pytest.mark.parametrize("H,res,wdt", [(1024, False, torch.bfloat16), (1024, True, torch.bfloat16),
                                       (960, True, torch.float32), (64, False, torch.float16)])
def test_rmsnorm_matches_oracle(H, res, wdt):
    dt = torch.float16 if wdt == torch.float16 else torch.bfloat16
    x = _rand(3, 101, H, seed=1, dtype=dt)
    r = _rand(3, 101, H, seed=2, scale=3.0, dtype=dt)
    w = (1 + 0.2 * _rand(H, seed=3, dtype=torch.float32)).to(wdt)
    with torch.inference_mode():
        out = epilogue.rmsnorm(x.to(DEV), w.to(DEV), 1e-6, residual=r.to(DEV) if res else None)
    torch.cuda.synchronize()
    if res:
        y, ro = out
        ry, rro = epilogue_ref.residual_rms_norm_ref(x, r, w, 1e-6)
        assert torch.equal(ro.cpu(), rro)
    else:
        y, ry = out, prologue_ref.rms_norm_ref(x, w, 1e-6)
    _ulp_ok(y, ry)


def test_add_rmsnorm_is_the_add_then_the_norm():
    # a bf16 torch add, then fla's RMSNorm of the rounded sum
    x = _rand(2, 333, 1024, seed=11)
    r = _rand(2, 333, 1024, seed=12, scale=4.0)
    w = (1 + 0.2 * _rand(1024, seed=13, dtype=torch.float32)).to(torch.bfloat16)
    with torch.inference_mode():
        y, h = epilogue.add_rmsnorm(x.to(DEV), r.to(DEV), w.to(DEV), 1e-6)
        want_h = r.to(DEV) + x.to(DEV)
    torch.cuda.synchronize()
    assert torch.equal(h, want_h)
    _ulp_ok(y, prologue_ref.rms_norm_ref(want_h.cpu(), w, 1e-6))


def test_swiglu_matches_oracle_on_strided_halves():
    gu = _rand(777, 2 * 3072, seed=4, scale=2.0)
    with torch.inference_mode():
        g = gu.to(DEV)
        z = ttt.swiglu(g[:, :3072], g[:, 3072:])
    torch.cuda.synchronize()
    _ulp_ok(z, R.swiglu_ref(gu[:, :3072], gu[:, 3072:]), pct=99.9)


FEAT = [
    # B, nchunk, C, I, K, conv_t, conv_s, w dtype
    pytest.param(1, 4, 256, 512, 5, True, True, torch.bfloat16, id="both-convs"),
    pytest.param(2, 3, 40, 64, 3, True, False, torch.float32, id="ragged-run-teacher-only-f32w"),
    pytest.param(1, 2, 64, 128, 5, False, True, torch.bfloat16, id="student-only"),
    pytest.param(1, 1, 96, 64, 5, True, True, torch.bfloat16, id="one-chunk"),
    pytest.param(1, 3, 32, 64, 1, False, False, torch.bfloat16, id="no-conv"),
]


@pytest.mark.parametrize("B,nchunk,C,I,K,ct,cs,wdt", FEAT)
def test_ttt_features_bitwise_chain(B, nchunk, C, I, K, ct, cs, wdt):
    """z within one rounding of the oracle's swiglu; z_hat and diff bit for bit
    equal to the oracle's conv and subtraction of the kernel's own swiglu
    values (a second call with the student rows on both sides yields them)."""
    rows = B * nchunk * C
    gu_t = _rand(rows, 2 * I, seed=5, scale=2.0)
    gu_s = _rand(rows, 2 * I, seed=6, scale=2.0)
    w_t = _rand(I, 1, K, seed=7, scale=0.5, dtype=wdt) if ct else None
    w_s = _rand(I, 1, K, seed=8, scale=0.5, dtype=wdt) if cs else None
    d = lambda v: None if v is None else v.to(DEV)  # noqa: E731
    with torch.inference_mode():
        z, zh, diff = ttt.ttt_features(gu_t.to(DEV), gu_s.to(DEV), d(w_t), d(w_s), B, nchunk, C)
        zr, _, _ = ttt.ttt_features(gu_s.to(DEV), gu_s.to(DEV), None, None, B, nchunk, C)
    torch.cuda.synchronize()
    _ulp_ok(z, R.swiglu_ref(gu_t[:, :I], gu_t[:, I:]), pct=99.9)
    z4, zr4 = z.cpu().reshape(B, nchunk, C, I), zr.cpu().reshape(B, nchunk, C, I)
    want_zh = R.conv_chunks(zr4, w_s).reshape(-1, I)
    assert torch.equal(zh.cpu(), want_zh)
    tgt = R.conv_chunks(z4, w_t)
    want_diff = (tgt[:, :nchunk - 1].float() - want_zh.reshape(B, nchunk, C, I)[:, :nchunk - 1]
                 .float()).to(z.dtype).reshape(-1, I)
    assert diff.shape == want_diff.shape and torch.equal(diff.cpu(), want_diff)


# ------------------------------------------------------------------ TTT MLP


def _ttt_setup(B, L, H, I, K, seed=0):
    g = torch.Generator().manual_seed(seed)

    def n(*s, std):
        return (torch.randn(*s, generator=g) * std).to(torch.bfloat16)
    w = ttt.TttMlpWeights(n(2 * I, H, std=H ** -0.5).to(DEV), n(H, I, std=I ** -0.5).to(DEV),
                          n(H, H, std=H ** -0.5).to(DEV), n(I, 1, K, std=0.4).to(DEV),
                          n(I, 1, K, std=0.4).to(DEV), n(H, std=H ** -0.5).to(DEV))
    x, t = n(B, L, H, std=1.0).to(DEV), n(B, L, H, std=1.0).to(DEV)
    return w, x, t


@pytest.mark.parametrize("B,L,C,G", [(1, 1024, 256, 16), (2, 700, 128, 2), (1, 256, 256, 4)])
def test_ttt_mlp_matches_oracle_loop(B, L, C, G):
    H, I, K = 256, 512, 5
    w, x, t = _ttt_setup(B, L, H, I, K, seed=B + L)
    with torch.inference_mode():
        y = ttt.ttt_mlp(x, t, w, chunk=C, lr=0.3, update_every=G)
        y2 = ttt.ttt_mlp(x, t, w, chunk=C, lr=0.3, update_every=G, fused=False)
        y3 = ttt.ttt_mlp(x, t, w, chunk=C, lr=0.3, update_every=G, scan="torch")
        # the oracle loop on the kernel's own features (same padding as the model)
        nch = -(-L // C)
        pad = nch * C - L
        xp = torch.nn.functional.pad(x, (0, 0, 0, pad))
        tp = torch.nn.functional.pad(t, (0, 0, 0, pad))
        gu = torch.nn.functional.linear(torch.cat([xp.reshape(-1, H), tp.reshape(-1, H)]),
                                        w.gate_up)
        rows = B * nch * C
        z, zh, diff = ttt.ttt_features(gu[:rows], gu[rows:], w.conv_t, w.conv_s, B, nch, C)
    torch.cuda.synchronize()
    # fused and separate feature passes are the same values, so the same output
    assert torch.equal(y, y2)
    # the scan kernels + batched GEMMs vs the reference's per-chunk torch ops:
    # the same roundings, the GEMMs' accumulation order may differ
    _logits_close(y, y3, max_frac=2e-2, mean_frac=1e-2)
    cpu = lambda v: v.cpu()  # noqa: E731
    want = R.ttt_mlp_scan_ref(cpu(z), cpu(zh), cpu(diff), cpu(tp), cpu(w.down), cpu(w.ttt_proj),
                              cpu(w.b_proj), lr=0.3, update_every=G, B=B, nchunk=nch, C=C)[:, :L]
    plain = (z.cpu().float() @ w.down.cpu().float().t()).reshape(B, nch * C, H)[:, :L]
    yf, wf = y.cpu().float(), want.float()
    rel = (yf - wf).norm() / wf.norm()
    assert rel < 1e-2, rel
    assert (yf - wf).abs().max() <= 3e-2 * wf.abs().max()
    if nch > 1:  # the update path is exercised: the output is not the plain MLP's
        assert (wf - plain).norm() / wf.norm() > 0.05


@pytest.mark.parametrize("B,K,C,H,dt,with_beta", [
    (1, 7, 256, 256, torch.bfloat16, True), (2, 3, 100, 72, torch.bfloat16, True),
    (1, 2, 64, 130, torch.float16, False)])
def test_proj_beta_t_is_torchs_multiply_transposed(B, K, C, H, dt, with_beta):
    """pd * beta (one rounding, the reference's bf16 multiply) written per chunk
    transposed, bit for bit against torch's own GPU ops."""
    pd = _rand(B * K * C, H, seed=K, scale=3.0, dtype=dt).to(DEV)
    beta = torch.sigmoid(_rand(B, K + 1, C, seed=C, dtype=torch.float32)).to(dt).to(DEV)
    with torch.inference_mode():
        got = ttt.proj_beta_t(pd, beta if with_beta else None, B, K, C)
        want = pd.view(B, K, C, H)
        if with_beta:
            want = want * beta[:, :K, :, None]
        want = want.transpose(-1, -2).reshape(B * K, H, C)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("nupd,nsteps,H,I,dt", [
    (7, 8, 256, 384, torch.bfloat16), (16, 16, 128, 256, torch.bfloat16),
    (3, 3, 100, 72, torch.bfloat16), (5, 6, 64, 200, torch.float16), (0, 1, 96, 64, torch.bfloat16)])
def test_scan_steps_are_torchs_bf16_scan(nupd, nsteps, H, I, dt):
    """The update scan of one group (scanfuse.py:157-170) against torch's own
    GPU ops, bit for bit: cumsum (a running sum stored in the dtype after
    every step), lr * cumsum, W_cur + cs for every chunk, the next W_cur; and
    torch's GPU cumsum against the oracle's step-wise scan."""
    dw = _rand(max(nupd, 1), H, I, seed=nupd + H, scale=2.0, dtype=dt)[:nupd].contiguous()
    w0 = _rand(H, I, seed=7, scale=0.05, dtype=dt)
    lr = 0.3
    with torch.inference_mode():
        steps, w_next = ttt.scan_steps(dw.to(DEV) if nupd else None, w0.to(DEV), lr, nsteps,
                                       want_next=nupd > 0)
        wc = w0.to(DEV)
        want = [wc]
        if nupd:
            csum = torch.cumsum(dw.to(DEV), dim=0)
            cs = torch.tensor(lr, dtype=dt, device=DEV) * csum
            want += [wc + cs[j] for j in range(nsteps - 1)]
            want_next = wc + cs[-1]
    torch.cuda.synchronize()
    assert steps.shape == (nsteps, I, H)
    for s_ in range(nsteps):
        assert torch.equal(steps[s_], want[s_].t()), s_
    if nupd:
        assert torch.equal(w_next, want_next)
        assert torch.equal(csum.cpu(), R.cumsum_stepwise(dw, 0))


# -------------------------------------------------------------------- model

TINY = dict(M.QWEN3_06B_SWA8K, hidden_size=256, num_hidden_layers=3, num_heads=4, num_kv_heads=2,
            head_dim=128, intermediate_size=512, vocab_size=1024, window_size=512,
            ttt_layers=[0, 2], ttt_chunk=256, ttt_update_every=2,
            ttt_teacher_conv_init="random", ttt_student_conv_init="random",
            max_position_embeddings=1024)


def _logits_close(got, want, max_frac=3e-2, mean_frac=2e-2):
    g, w = got.float().cpu(), want.float().cpu()
    d = (g - w).abs()
    assert d.max() <= max_frac * w.abs().max(), (d.max(), w.abs().max())
    assert d.mean() <= mean_frac * w.abs().mean(), (d.mean(), w.abs().mean())


@pytest.mark.parametrize("T", [1024, 900, 200])
def test_prefill_matches_oracle(T):
    """T=1024: 4 chunks in 2 update groups; T=900: a zero-padded last chunk;
    T=200: shorter than a chunk, so the TTT layers take the plain path."""
    c = M.resolve_config(TINY)
    w = M.init_weights(TINY, DEV, seed=0)
    ids = torch.randint(0, c["vocab_size"], (1, T), generator=torch.Generator().manual_seed(T))
    got = {p: M.IPTTCDv9Prefill(TINY, w, path=p).forward(ids.to(DEV), logits_to_keep=8)
           for p in M.PATHS}
    torch.cuda.synchronize()
    want = R.prefill_ref(c, {k: v.cpu() for k, v in w.items()}, ids, 8, torch.bfloat16)
    for p in M.PATHS:
        _logits_close(got[p], want)
    # the patches change only rounding
    _logits_close(got["fused"], got["stock"], max_frac=2e-2, mean_frac=1e-2)
    _logits_close(got["fused"], got["patched"], max_frac=2e-2, mean_frac=1e-2)


def test_patch_hooks_turn_stock_into_patched():
    w = M.init_weights(TINY, DEV, seed=3)
    model = M.IPTTCDv9Prefill(TINY, w, path="stock")
    assert model.path == "stock"
    assert M.patch_fused_attn(model) == 2 and M.patch_triton_conv(model) == 2
    assert model.path == "patched"
    ids = torch.randint(0, 1024, (1, 768), generator=torch.Generator().manual_seed(11)).to(DEV)
    a = model.forward(ids, logits_to_keep=4)
    b = M.IPTTCDv9Prefill(TINY, w, path="patched").forward(ids, logits_to_keep=4)
    M.patch_fused_attn(model, kernel="fa3_lse")
    lse = model.forward(ids, logits_to_keep=4)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    _logits_close(lse, a, max_frac=2e-2, mean_frac=1e-2)


# SmolLM2-360M's attention shape (configs/ipttcd/ipttcdv9_smollm2_360M_ct_64k_v2_swa8k.json):
# 15 query / 5 KV heads of 64, no qk_norm, rope_theta 1e5, norm_eps 1e-5
SMOL = dict(TINY, hidden_size=960, num_heads=15, num_kv_heads=5, head_dim=64, qk_norm=False,
            rope_theta=100000.0, norm_eps=1e-05, intermediate_size=640, ttt_layers=[1])


def test_prefill_smollm2_shape_matches_oracle():
    c = M.resolve_config(SMOL)
    w = M.init_weights(SMOL, DEV, seed=2)
    model = M.IPTTCDv9Prefill(SMOL, w)
    ids = torch.randint(0, c["vocab_size"], (1, 768), generator=torch.Generator().manual_seed(7))
    got = model.forward(ids.to(DEV), logits_to_keep=8)
    torch.cuda.synchronize()
    want = R.prefill_ref(c, {k: v.cpu() for k, v in w.items()}, ids, 8, torch.bfloat16)
    _logits_close(got, want)


def test_prefill_batch_rows_are_independent():
    c = M.resolve_config(TINY)
    w = M.init_weights(TINY, DEV, seed=1)
    model = M.IPTTCDv9Prefill(TINY, w)
    ids = torch.randint(0, c["vocab_size"], (2, 512), generator=torch.Generator().manual_seed(9))
    both = model.forward(ids.to(DEV), logits_to_keep=4)
    one = model.forward(ids[1:].to(DEV), logits_to_keep=4)
    torch.cuda.synchronize()
    _logits_close(both[1:], one, max_frac=1e-2, mean_frac=5e-3)


@torch.inference_mode()
def test_config5_full_size_paths_agree():
    """Config 5 at its full size: the Qwen3-0.6B-shaped ipttcdv9 (28 layers,
    TTT layers 0/7/14/21, vocab 151936), weights N(0, 0.02) from seed 0, T=32768
    uniform token ids (seed 1234), as bench.py's e2e measurement runs it. A
    CPU oracle of 28 layers at 32K tokens does not finish in a test's time, so
    the size-independent checks: every path's logits are finite, and the
    patched and fused paths agree with the stock path (the reference's
    unpatched fast prefill: two windowed calls and torch's conv) within the
    bounds the small configs hold against the oracle."""
    cfg = M.QWEN3_06B_SWA8K
    print("config 5: ipttcdv9 Qwen3-0.6B shape, T=32768", flush=True)
    w = M.init_weights(cfg, DEV, seed=0)
    g = torch.Generator(device=DEV).manual_seed(1234)
    ids = torch.randint(0, cfg["vocab_size"], (1, 32768), device=DEV, generator=g)
    got = {}
    for p in M.PATHS:
        got[p] = M.IPTTCDv9Prefill(cfg, w, path=p).forward(ids, logits_to_keep=8)
        torch.cuda.synchronize()
        assert got[p].shape == (1, 8, cfg["vocab_size"])
        assert got[p].isfinite().all(), p
    _logits_close(got["fused"], got["stock"])
    _logits_close(got["patched"], got["stock"])
    _logits_close(got["fused"], got["patched"], max_frac=2e-2, mean_frac=1e-2)


# ------------------------------------------------ fast-path gate and fallback

def _ids(B, T, seed, vocab=1024):
    return torch.randint(0, vocab, (B, T), generator=torch.Generator().manual_seed(seed))


def test_disabled_fast_path_matches_fast_path_and_oracle(monkeypatch):
    """IPTTCD_DISABLE_FAST_PREFILL=1 routes the TTT layers through the
    reference's fallback (two windowed calls, two norms;
    modeling_ipttcdv9.py:562-574, 794-850), which the reference calls bit-exact
    with its fast path: here both match the oracle and each other."""
    c = M.resolve_config(TINY)
    w = M.init_weights(TINY, DEV, seed=4)
    ids = _ids(1, 1024, 41)
    fast = M.IPTTCDv9Prefill(TINY, w).forward(ids.to(DEV), logits_to_keep=8)
    monkeypatch.setenv("IPTTCD_DISABLE_FAST_PREFILL", "1")
    slow = M.IPTTCDv9Prefill(TINY, w).forward(ids.to(DEV), logits_to_keep=8)
    torch.cuda.synchronize()
    want = R.prefill_ref(c, {k: v.cpu() for k, v in w.items()}, ids, 8, torch.bfloat16)
    _logits_close(slow, want)
    _logits_close(fast, slow, max_frac=2e-2, mean_frac=1e-2)


def test_padding_mask_takes_the_fallback_and_matches_oracle():
    """A left-padded batch: every layer attends within each row's unpadded
    tokens (fla Attention's varlen path), the TTT student over the whole
    row, as the reference's fallback does."""
    c = M.resolve_config(TINY)
    w = M.init_weights(TINY, DEV, seed=5)
    B, T = 2, 1024
    ids = _ids(B, T, 51)
    mask = torch.ones(B, T, dtype=torch.long)
    mask[0, :200] = 0          # row 0 left-padded by 200 tokens
    got = M.IPTTCDv9Prefill(TINY, w).forward(ids.to(DEV), logits_to_keep=8,
                                             attention_mask=mask.to(DEV))
    torch.cuda.synchronize()
    want = R.prefill_ref(c, {k: v.cpu() for k, v in w.items()}, ids, 8, torch.bfloat16,
                         attention_mask=mask)
    _logits_close(got, want)
    # a mask of ones is no mask: the fast path
    ones = M.IPTTCDv9Prefill(TINY, w).forward(ids.to(DEV), logits_to_keep=8,
                                              attention_mask=torch.ones_like(mask).to(DEV))
    none = M.IPTTCDv9Prefill(TINY, w).forward(ids.to(DEV), logits_to_keep=8)
    torch.cuda.synchronize()
    assert torch.equal(ones, none)


def test_packed_sequences_take_the_fallback_and_match_oracle():
    """cu_seqlens: three sequences packed in one row; attention within each,
    rotary positions restarting per sequence, the TTT student over the row."""
    c = M.resolve_config(TINY)
    w = M.init_weights(TINY, DEV, seed=6)
    ids = _ids(1, 1024, 61)
    cu = torch.tensor([0, 300, 701, 1024], dtype=torch.int32)
    got = M.IPTTCDv9Prefill(TINY, w).forward(ids.to(DEV), logits_to_keep=8,
                                             cu_seqlens=cu.to(DEV))
    torch.cuda.synchronize()
    want = R.prefill_ref(c, {k: v.cpu() for k, v in w.items()}, ids, 8, torch.bfloat16,
                         cu_seqlens=cu)
    _logits_close(got, want)


# MHA so that fla's g_proj (num_kv_heads * head_dim outputs) matches the output
GATED = dict(TINY, num_kv_heads=4, use_output_gate=True)


@pytest.mark.parametrize("gate_fn", ["sigmoid", "swish"])
def test_output_gate_on_every_path_matches_oracle(gate_fn):
    """use_output_gate (fla/layers/attn.py:284-292) on the stock, patched and
    fused paths, and on the fallback. The reference's patched forward drops
    the gate (strict xfail, test/test_fused_dual_attn.py:339-360); here every
    path applies it to both attention outputs. gate_fn 'swish' with fuse_norm
    is FusedRMSNormGated."""
    cfg = dict(GATED, gate_fn=gate_fn)
    c = M.resolve_config(cfg)
    w = M.init_weights(cfg, DEV, seed=7)
    # non-trivial gate norm weights
    for key in list(w):
        if key.endswith(("g_norm.weight", "g_norm_swish_gate.weight")):
            w[key] = (1 + 0.3 * _rand(w[key].shape[0], seed=len(key))).to(DEV)
    ids = _ids(1, 1024, 71)
    want = R.prefill_ref(c, {k: v.cpu() for k, v in w.items()}, ids, 8, torch.bfloat16)
    got = {p: M.IPTTCDv9Prefill(cfg, w, path=p).forward(ids.to(DEV), logits_to_keep=8)
           for p in M.PATHS}
    torch.cuda.synchronize()
    for p in M.PATHS:
        _logits_close(got[p], want)
    # the gate matters: without it the logits move
    plain = R.prefill_ref(dict(c, use_output_gate=False), {k: v.cpu() for k, v in w.items()},
                          ids, 8, torch.bfloat16)
    assert (plain.float() - want.float()).abs().mean() > 0.1 * want.float().abs().mean()


@pytest.mark.parametrize("chunks", [(600, 300), (300, 700, 256)])
def test_prefill_in_chunks_over_the_cache_matches_oracle(chunks):
    """A prompt prefilled in chunks over IPTTCDv9Cache (the attention kernels'
    Tq < Tk forms, the window-trimmed per-layer K/V, the rotary offset) against
    the oracle's chunked prefill, every path. Every chunk has at least one TTT
    chunk (256 tokens), so the TTT layers run the dual-window kernel on
    Tq < Tk; (600, 300): the first chunk already fills the 512-token window,
    so the cache is trimmed before the second; (300, 700, 256): the cache
    grows, then is trimmed, and the last chunk is exactly one TTT chunk."""
    c = M.resolve_config(TINY)
    w = M.init_weights(TINY, DEV, seed=9)
    wc = {k: v.cpu() for k, v in w.items()}
    T = sum(chunks)
    ids = torch.randint(0, c["vocab_size"], (1, T), generator=torch.Generator().manual_seed(T))
    for p in M.PATHS:
        model = M.IPTTCDv9Prefill(TINY, w, path=p)
        cache, rcache = M.IPTTCDv9Cache(), R.new_cache_ref()
        a = 0
        for n in chunks:
            print(f"path {p}: chunk {a}..{a + n}", flush=True)
            got = model.forward(ids[:, a:a + n].to(DEV), logits_to_keep=8, cache=cache)
            torch.cuda.synchronize()
            want = R.prefill_ref(c, wc, ids[:, a:a + n], 8, torch.bfloat16, cache=rcache)
            _logits_close(got, want)
            a += n
            assert cache.seen == a
            assert cache.kv[0][0].shape[1] == min(a, TINY["window_size"])


def test_prefill_in_chunks_equals_one_prefill_without_ttt():
    """With no TTT layer (the TTT MLP restarts per chunk), a chunked prefill's
    logits equal one prefill of the whole prompt on every row."""
    cfg = dict(TINY, ttt_layers=[])
    w = M.init_weights(cfg, DEV, seed=10)
    model = M.IPTTCDv9Prefill(cfg, w)
    ids = _ids(1, 1000, seed=11).to(DEV)
    whole = model.forward(ids, logits_to_keep=0)
    cache, a = M.IPTTCDv9Cache(), 0
    for n in (450, 50, 500):
        part = model.forward(ids[:, a:a + n], logits_to_keep=0, cache=cache)
        _logits_close(part, whole[:, a:a + n], max_frac=2e-2, mean_frac=1e-2)
        a += n
