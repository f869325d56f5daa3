"""ipttcdv9 prefill, CPU side: the model oracle pinned against an independent
implementation (transformers' Qwen3, which a TTT-free full-causal ipttcdv9 is)
and the TTT MLP's two formulations against each other; config resolution;
the C ABI's argument checks for the new entry points (before any HIP call)."""
from __future__ import annotations

import ctypes

import pytest
import torch

from oracle import attn_ref, ipttcdv9_ref as R
from ttcd_amd import _lib, ipttcdv9 as M

TINY = dict(M.QWEN3_06B_SWA8K, hidden_size=256, num_hidden_layers=3, num_heads=4, num_kv_heads=2,
            head_dim=64, intermediate_size=512, vocab_size=1024, window_size=512,
            ttt_layers=[0, 2], ttt_chunk=256, ttt_update_every=2,
            ttt_teacher_conv_init="random", ttt_student_conv_init="random",
            max_position_embeddings=1024)


def _rand(*shape, seed=0, scale=1.0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


# ------------------------------------------------------------ TTT MLP pins


def _scan_inputs(B, nchunk, C, I, H, seed=0):
    z = _rand(B * nchunk * C, I, seed=seed)
    zh = _rand(B * nchunk * C, I, seed=seed + 1)
    diff = _rand(B * (nchunk - 1) * C, I, seed=seed + 2)
    t = _rand(B, nchunk * C, H, seed=seed + 3)
    wd = _rand(H, I, seed=seed + 4, scale=0.1)
    P = _rand(H, H, seed=seed + 5, scale=0.3)
    bp = _rand(H, seed=seed + 6, scale=0.3)
    return z, zh, diff, t, wd, P, bp


@pytest.mark.parametrize("B,nchunk,update_every", [(1, 2, 16), (2, 5, 16), (2, 5, 2), (1, 6, 1),
                                                   (1, 7, 3), (1, 1, 4)])
def test_scan_equals_per_token_form(B, nchunk, update_every):
    C, I, H = 8, 16, 12
    z, zh, diff, t, wd, P, bp = _scan_inputs(B, nchunk, C, I, H)
    got = R.ttt_mlp_scan_ref(z, zh, diff, t, wd, P, bp, lr=0.3, update_every=update_every,
                             B=B, nchunk=nchunk, C=C, dt=torch.float64)
    want = R.ttt_mlp_token_f64(z, zh, diff, t, wd, P, bp, lr=0.3, B=B, nchunk=nchunk, C=C)
    assert torch.allclose(got, want, rtol=1e-10, atol=1e-10)


def test_planted_off_by_one_fails_the_pin():
    # a chunk that also used its own update (W for chunk c = W_cur + cs[c])
    B, nchunk, C, I, H = 1, 4, 8, 16, 12
    z, zh, diff, t, wd, P, bp = _scan_inputs(B, nchunk, C, I, H, seed=3)
    want = R.ttt_mlp_token_f64(z, zh, diff, t, wd, P, bp, lr=0.3, B=B, nchunk=nchunk, C=C)
    # token form with the mistake: acc updated before the chunk's output
    Wu = wd.t() @ P
    beta = torch.sigmoid(t[0] @ bp)
    acc = wd.clone()
    wrong = torch.empty_like(want)
    for c in range(nchunk):
        rows = slice(c * C, (c + 1) * C)
        if c < nchunk - 1:
            upd = sum(torch.outer(beta[s] * (diff[s] @ Wu), zh[s]) for s in range(c * C, (c + 1) * C))
            acc = acc + 0.3 * upd
        wrong[0, rows] = z[rows] @ acc.t()
    assert not torch.allclose(wrong, want, rtol=1e-6, atol=1e-6)


def test_lr_zero_and_no_difference_reduce_to_the_plain_mlp():
    B, nchunk, C, I, H = 2, 3, 8, 16, 12
    z, zh, diff, t, wd, P, bp = _scan_inputs(B, nchunk, C, I, H, seed=5)
    plain = (z @ wd.t()).reshape(B, nchunk * C, H)
    got = R.ttt_mlp_scan_ref(z, zh, diff, t, wd, P, bp, lr=0.0, update_every=16, B=B,
                             nchunk=nchunk, C=C, dt=torch.float64)
    assert torch.allclose(got, plain, rtol=1e-12, atol=1e-12)
    got = R.ttt_mlp_scan_ref(z, zh, torch.zeros_like(diff), t, wd, P, bp, lr=0.3,
                             update_every=16, B=B, nchunk=nchunk, C=C, dt=torch.float64)
    assert torch.allclose(got, plain, rtol=1e-12, atol=1e-12)


def test_cumsum_stepwise_rounds_every_step():
    # bf16 ulp at 1 is 2^-7: 1 + 3*2^-10 rounds back to 1 each step, while an
    # fp32 running sum reaches 1 + 6*2^-10 and rounds up at the end
    x = torch.tensor([1.0, 3 * 2**-10, 3 * 2**-10]).to(torch.bfloat16)
    got = R.cumsum_stepwise(x)
    assert got.tolist() == [1.0, 1.0, 1.0]
    assert torch.cumsum(x.float(), 0).to(torch.bfloat16)[-1].item() == 1.0078125
    # exact sums are left alone
    y = torch.tensor([1.0, 2.0, -0.5, 4.0]).to(torch.bfloat16)
    assert torch.equal(R.cumsum_stepwise(y), torch.cumsum(y.float(), 0).to(torch.bfloat16))


def test_swiglu_ref_within_one_rounding():
    g = _rand(4096, seed=7, scale=3.0, dtype=torch.bfloat16)
    u = _rand(4096, seed=8, scale=2.0, dtype=torch.bfloat16)
    got = R.swiglu_ref(g, u)
    gd, ud = g.double(), u.double()
    want = (gd / (1 + torch.exp(-gd)) * ud).float().to(torch.bfloat16)
    rep = attn_ref.ulp_report(got, want)
    assert rep["max_ulp"] <= 1 and rep["bit_equal_pct"] > 99.5, rep


def test_features_ref_diff_of_stored_values():
    B, nchunk, C, I = 1, 3, 16, 32
    gu_t = _rand(B * nchunk * C, 2 * I, seed=9, dtype=torch.bfloat16)
    gu_s = _rand(B * nchunk * C, 2 * I, seed=10, dtype=torch.bfloat16)
    cw = _rand(I, 1, 5, seed=11, scale=0.5, dtype=torch.bfloat16)
    z, zh, diff = R.ttt_features_ref(gu_t, gu_s, cw, cw, B, nchunk, C)
    # same input and same conv on both sides: zero difference
    z2, zh2, d2 = R.ttt_features_ref(gu_t, gu_t, cw, cw, B, nchunk, C)
    assert torch.all(d2 == 0)
    # no conv: z_hat is the student swiglu, diff its difference from z
    _, zh3, d3 = R.ttt_features_ref(gu_t, gu_s, None, None, B, nchunk, C)
    assert torch.equal(zh3, R.swiglu_ref(gu_s[:, :I], gu_s[:, I:]))
    assert diff.shape == (B * (nchunk - 1) * C, I)


# ------------------------------------------------------- model oracle pin


def test_prefill_ref_matches_transformers_qwen3():
    """A TTT-free ipttcdv9 with full causal attention is Qwen3: the oracle's
    norms, projections, GQA, rotary, SwiGLU and tied head against
    transformers' own implementation, in float32."""
    from transformers import Qwen3Config, Qwen3ForCausalLM

    cfg = dict(TINY, num_hidden_layers=2, ttt_mode=False, window_size=None, norm_eps=1e-5,
               rope_theta=1e6)
    c = M.resolve_config(cfg)
    w = {k: v.float() for k, v in M.init_weights(cfg, "cpu", torch.float32, seed=0).items()}
    # random norm weights so a missed weight would show
    g = torch.Generator().manual_seed(3)
    for k in list(w):
        if k.endswith("norm.weight"):
            w[k] = 1 + 0.2 * torch.randn(w[k].shape, generator=g)
    hc = Qwen3Config(vocab_size=c["vocab_size"], hidden_size=c["hidden_size"],
                     intermediate_size=c["intermediate_size"],
                     num_hidden_layers=c["num_hidden_layers"], num_attention_heads=c["num_heads"],
                     num_key_value_heads=c["num_kv_heads"], head_dim=c["head_dim"],
                     rms_norm_eps=1e-5, rope_theta=1e6, max_position_embeddings=1024,
                     tie_word_embeddings=True, attention_bias=False, use_sliding_window=False)
    hc._attn_implementation = "eager"
    model = Qwen3ForCausalLM(hc).float().eval()
    sd = {"model.embed_tokens.weight": w["model.embeddings.weight"],
          "model.norm.weight": w["model.norm.weight"], "lm_head.weight": w["lm_head.weight"]}
    for i in range(c["num_hidden_layers"]):
        p, q = f"model.layers.{i}.", f"model.layers.{i}."
        sd[q + "input_layernorm.weight"] = w[p + "attn_norm.weight"]
        sd[q + "post_attention_layernorm.weight"] = w[p + "mlp_norm.weight"]
        for n in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm"):
            sd[q + f"self_attn.{n}.weight"] = w[p + f"attn.{n}.weight"]
        for n in ("gate_proj", "up_proj", "down_proj"):
            sd[q + f"mlp.{n}.weight"] = w[p + f"mlp.{n}.weight"]
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    ids = torch.randint(0, c["vocab_size"], (2, 200), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        want = model(input_ids=ids).logits[:, -5:].float()
    got = R.prefill_ref(c, w, ids, 5, torch.float32)
    assert torch.allclose(got, want, rtol=1e-3, atol=2e-4), (got - want).abs().max()


def test_prefill_ref_window_changes_the_result_only_past_the_window():
    cfg = dict(TINY, num_hidden_layers=1, ttt_mode=False, window_size=64)
    c = M.resolve_config(cfg)
    w = {k: v.float() for k, v in M.init_weights(cfg, "cpu", torch.float32, seed=1).items()}
    ids = torch.randint(0, c["vocab_size"], (1, 160), generator=torch.Generator().manual_seed(5))
    full = M.resolve_config(dict(cfg, window_size=None))
    a = R.prefill_ref(c, w, ids, 160, torch.float32)
    b = R.prefill_ref(full, w, ids, 160, torch.float32)
    assert torch.allclose(a[:, :64], b[:, :64], rtol=1e-5, atol=1e-6)
    assert not torch.allclose(a[:, 100:], b[:, 100:], rtol=1e-3, atol=1e-4)


# ------------------------------------------------------- config and FLOPs


def test_resolve_config_and_unsupported_options():
    c = M.resolve_config(M.QWEN3_06B_SWA8K)
    assert (c["intermediate_size"], c["head_dim"], c["ttt_layers"]) == (3072, 128, [0, 7, 14, 21])
    assert c["ttt_visible_chunks"] * c["ttt_chunk"] == 4096
    derived = M.resolve_config({"hidden_size": 1024, "num_heads": 16, "vocab_size": 10,
                                "num_hidden_layers": 1})
    # modeling_ipttcdv9.py:98-102: 256 * ceil(1024 * 4 * 2 / 3 / 256)
    assert derived["intermediate_size"] == 2816 and derived["head_dim"] == 64
    for bad in ({"ttt_weight_renorm": True}, {"use_muon": True},
                {"ttt_normalize_student_features": True}, {"qkv_bias": True},
                {"fuse_norm": False}, {"ttt_scan_state_dtype": "fp32"},
                {"ttt_scan_state_dtype": "BF16"}):
        with pytest.raises(NotImplementedError):
            M.resolve_config(dict(M.QWEN3_06B_SWA8K, **bad))


def test_init_weights_follow_the_reference_init():
    w = M.init_weights(TINY, "cpu", seed=0)
    p = "model.layers.0.mlp."
    P = w[p + "ttt_proj.weight"].float()
    assert torch.equal(P, torch.diag(torch.diagonal(P)))          # diagonal_gaussian
    assert torch.all(w["model.layers.0.attn_norm.weight"] == 1)
    assert w["lm_head.weight"] is w["model.embeddings.weight"]     # tied
    ident = M.init_weights(dict(TINY, ttt_teacher_conv_init="identity",
                                ttt_student_conv_init="zero"), "cpu", seed=0)
    tc = ident[p + "ttt_teacher_conv.weight"].float()
    assert torch.all(tc[:, 0, -1] == 1) and torch.all(tc[:, 0, :-1] == 0)
    assert torch.all(ident[p + "ttt_student_conv.weight"] == 0)
    assert "model.layers.1.mlp.ttt_proj.weight" not in w


def test_prefill_flops():
    f = M.prefill_flops(M.QWEN3_06B_SWA8K, 1, 32768)
    # 28 teacher bands of 4*16*128*P(32768, 8192)
    P = 8192 * 8193 // 2 + (32768 - 8192) * 8192
    assert f["attention"] == 28 * 4 * 16 * 128 * P
    assert 3.2e13 < f["gemm"] < 3.3e13


# ------------------------------------------------------------ C ABI checks

_P = ctypes.c_void_p(0x10000)


def test_rmsnorm_abi_rejects():
    L = _lib.lib()
    ok = dict(x=_P, r=None, w=_P, wdt=_lib.DTYPE_BF16, eps=1e-6, y=_P, ro=None, rows=4, H=64,
              dt=_lib.DTYPE_BF16)

    def call(**o):
        a = dict(ok, **o)
        return L.ttcd_rmsnorm_fwd(a["x"], a["r"], a["w"], a["wdt"], a["eps"], a["y"], a["ro"],
                                  a["rows"], a["H"], a["dt"], None)
    assert call(x=None) == _lib.TTCD_ERR_INVALID_ARGUMENT
    assert call(r=_P) == _lib.TTCD_ERR_INVALID_ARGUMENT          # residual without residual_out
    assert call(H=60) == _lib.TTCD_ERR_UNSUPPORTED
    assert call(eps=-1.0) == _lib.TTCD_ERR_INVALID_ARGUMENT
    assert call(y=ctypes.c_void_p(0x10008)) == _lib.TTCD_ERR_UNSUPPORTED
    assert call(rows=0) == _lib.TTCD_OK


def test_add_rmsnorm_abi_rejects():
    L = _lib.lib()
    args = [_P, _P, _P, _lib.DTYPE_BF16, 1e-6, _P, _P, 4, 64, _lib.DTYPE_BF16, None]
    bad = list(args); bad[1] = None
    assert L.ttcd_add_rmsnorm_fwd(*bad) == _lib.TTCD_ERR_INVALID_ARGUMENT
    bad = list(args); bad[8] = 2056
    assert L.ttcd_add_rmsnorm_fwd(*bad) == _lib.TTCD_ERR_UNSUPPORTED
    bad = list(args); bad[6] = ctypes.c_void_p(0x10008)
    assert L.ttcd_add_rmsnorm_fwd(*bad) == _lib.TTCD_ERR_UNSUPPORTED
    ok = list(args); ok[7] = 0
    assert L.ttcd_add_rmsnorm_fwd(*ok) == _lib.TTCD_OK


def test_swiglu_abi_rejects():
    L = _lib.lib()
    assert L.ttcd_swiglu_fwd(None, _P, _P, 4, 64, 64, 64, 64, _lib.DTYPE_BF16, None) == \
        _lib.TTCD_ERR_INVALID_ARGUMENT
    assert L.ttcd_swiglu_fwd(_P, _P, _P, 4, 64, 32, 64, 64, _lib.DTYPE_BF16, None) == \
        _lib.TTCD_ERR_INVALID_ARGUMENT
    assert L.ttcd_swiglu_fwd(_P, _P, _P, 4, 60, 64, 64, 64, _lib.DTYPE_BF16, None) == \
        _lib.TTCD_ERR_UNSUPPORTED
    assert L.ttcd_swiglu_fwd(_P, _P, _P, 4, 64, 64, 64, 64, _lib.DTYPE_F32, None) == \
        _lib.TTCD_ERR_UNSUPPORTED
    assert L.ttcd_swiglu_fwd(_P, _P, _P, 0, 64, 64, 64, 64, _lib.DTYPE_BF16, None) == _lib.TTCD_OK


def test_ttt_features_abi_rejects():
    L = _lib.lib()

    def call(gu=_P, st=128, cw=_P, K=5, diff=_P, nch=4, inter=64, dt=_lib.DTYPE_BF16):
        return L.ttcd_ttt_features_fwd(gu, _P, st, cw, cw, _lib.DTYPE_BF16, K, _P, _P, diff,
                                       1, nch, 16, inter, dt, None)
    assert call(gu=None) == _lib.TTCD_ERR_INVALID_ARGUMENT
    assert call(diff=None) == _lib.TTCD_ERR_INVALID_ARGUMENT
    assert call(st=100) == _lib.TTCD_ERR_INVALID_ARGUMENT
    assert call(K=9) == _lib.TTCD_ERR_UNSUPPORTED
    assert call(inter=60, st=120) == _lib.TTCD_ERR_UNSUPPORTED
    assert call(dt=_lib.DTYPE_F32) == _lib.TTCD_ERR_UNSUPPORTED
    assert call(gu=ctypes.c_void_p(0x10008)) == _lib.TTCD_ERR_UNSUPPORTED


def test_python_layers_refuse_cpu_tensors():
    from ttcd_amd import epilogue, ttt
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        epilogue.rmsnorm(x, torch.ones(64), 1e-6)
    with pytest.raises(ValueError, match="GPU"):
        ttt.swiglu(x, x)


def test_output_gate_config_rules():
    # fla's g_proj has num_kv_heads * head_dim outputs: the gate needs MHA
    with pytest.raises(ValueError):
        M.resolve_config(dict(M.QWEN3_06B_SWA8K, use_output_gate=True))
    c = M.resolve_config(dict(M.QWEN3_06B_SWA8K, use_output_gate=True, num_kv_heads=16))
    assert c["gate_fn"] == "sigmoid"
    with pytest.raises(NotImplementedError):
        M.resolve_config(dict(M.QWEN3_06B_SWA8K, use_output_gate=True, num_kv_heads=16,
                              gate_fn="relu"))
    with pytest.raises(NotImplementedError):
        M.resolve_config(dict(M.QWEN3_06B_SWA8K, use_l2_softmax=True))
    w = M.init_weights(dict(TINY, num_kv_heads=4, use_output_gate=True, gate_fn="swish"), "cpu")
    assert "model.layers.0.attn.g_proj.weight" in w
    assert "model.layers.0.attn.g_norm_swish_gate.weight" in w


def test_oracle_packed_sequences_equal_each_sequence_alone():
    """The oracle's cu_seqlens path (per-sequence attention, rotary positions
    restarting per sequence) on a TTT-free config gives each sequence the
    logits of a prefill of that sequence alone."""
    cfg = dict(TINY, ttt_layers=[], num_hidden_layers=2)
    c = M.resolve_config(cfg)
    w = M.init_weights(cfg, "cpu", seed=2)
    ids = torch.randint(0, 1024, (1, 96), generator=torch.Generator().manual_seed(3))
    cu = torch.tensor([0, 40, 96])
    packed = R.prefill_ref(c, w, ids, 0, torch.float32, cu_seqlens=cu)
    for a, b in ((0, 40), (40, 96)):
        alone = R.prefill_ref(c, w, ids[:, a:b], 0, torch.float32)
        torch.testing.assert_close(packed[:, a:b], alone, rtol=1e-4, atol=1e-4)


def test_oracle_padding_mask_equals_unpadded_row_up_to_rope_positions():
    """A right-padded row under the mask equals the same tokens alone (right
    padding keeps the rotary positions), on a TTT-free config."""
    cfg = dict(TINY, ttt_layers=[], num_hidden_layers=2)
    c = M.resolve_config(cfg)
    w = M.init_weights(cfg, "cpu", seed=4)
    ids = torch.randint(0, 1024, (1, 80), generator=torch.Generator().manual_seed(5))
    mask = torch.ones(1, 80, dtype=torch.long)
    mask[0, 50:] = 0
    masked = R.prefill_ref(c, w, ids, 0, torch.float32, attention_mask=mask)
    alone = R.prefill_ref(c, w, ids[:, :50], 0, torch.float32)
    torch.testing.assert_close(masked[:, :50], alone, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("window,chunks", [(64, (100, 60, 40)), (None, (70, 50)),
                                           (64, (30, 20, 110))])
def test_oracle_chunked_prefill_equals_one_shot(window, chunks):
    """A prompt prefilled in chunks over the oracle's K/V cache gives every row
    the logits of one prefill of the whole prompt, on a TTT-free config (the TTT
    MLP restarts per chunk): the rotary offset continues, each chunk attends
    over the kept keys, and a cache trimmed to the window (first case) still
    holds every key the next chunk's window reaches."""
    cfg = dict(TINY, ttt_layers=[], num_hidden_layers=2, window_size=window)
    c = M.resolve_config(cfg)
    w = M.init_weights(cfg, "cpu", seed=6)
    T = sum(chunks)
    ids = torch.randint(0, 1024, (2, T), generator=torch.Generator().manual_seed(7))
    whole = R.prefill_ref(c, w, ids, 0, torch.float32)
    cache = R.new_cache_ref()
    a = 0
    for n in chunks:
        part = R.prefill_ref(c, w, ids[:, a:a + n], 0, torch.float32, cache=cache)
        torch.testing.assert_close(part, whole[:, a:a + n], rtol=1e-4, atol=1e-4)
        a += n
        assert cache["seen"] == a
        kept = cache["kv"][0][0].shape[1]
        assert kept == (a if window is None else min(window, a))


def test_oracle_chunked_prefill_detects_planted_offset_mistake():
    """Planted mistake: the second chunk's rotary positions restart at 0 (the
    cache's token count dropped) -- its logits must move off the one-shot ones."""
    cfg = dict(TINY, ttt_layers=[], num_hidden_layers=2, window_size=64)
    c = M.resolve_config(cfg)
    w = M.init_weights(cfg, "cpu", seed=6)
    ids = torch.randint(0, 1024, (1, 120), generator=torch.Generator().manual_seed(8))
    whole = R.prefill_ref(c, w, ids, 0, torch.float32)
    cache = R.new_cache_ref()
    R.prefill_ref(c, w, ids[:, :80], 0, torch.float32, cache=cache)
    cache["seen"] = 0
    bad = R.prefill_ref(c, w, ids[:, 80:], 0, torch.float32, cache=cache)
    assert (bad - whole[:, 80:]).abs().max().item() > 1e-2
