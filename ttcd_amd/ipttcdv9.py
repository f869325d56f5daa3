"""Prefill of an ipttcdv9 (IP-TTCD) model on gfx950, end to end.

A forward-only restatement of IPTTCDForCausalLM's prefill
(custom_models/ipttcd/modeling_ipttcdv9.py:577-880, 999-1128, 1194-1241),
with the TTT MLP of modeling_ipttcdv9_lowcopy_scanfuse.py:36-204 (what
profiling/bench_prefill.py runs by default) and the two patches that
`bench_prefill.py --patch fused_conv` installs (profiling/patches.py:
215-312 fused dual-window attention on the TTT layers, 411-432 chunk-local
conv). It runs no reference code: parameters are held under the reference's
state-dict names, and every step calls this package's HIP kernels or a
hipBLASLt GEMM through torch.

Per layer (attn_norm = fla RMSNorm; qk_norm + rotary; window W_T):
  plain layer: h -> RMSNorm -> one q|k|v GEMM -> q/k RMSNorm + rotary (one
      kernel) -> band attention (window W_T) -> o_proj -> residual RMSNorm
      -> gate|up GEMM -> SwiGLU -> down GEMM -> residual add (one kernel with
      the next block's RMSNorm, the sum rounded first as the reference's add)
  TTT layer:   ... -> fused dual-window attention (W_T, W_S = visible chunks
      x ttt_chunk) -> one o_proj GEMM over both outputs -> dual residual
      RMSNorm -> TTT MLP (ttcd_amd.ttt.ttt_mlp) -> residual add
then the final RMSNorm and the LM head on the last `logits_to_keep` tokens.

Three paths for the TTT layers, chosen per model (`path=`) or by the
patches-shaped hooks below, the same A/B as `bench_prefill.py --patch none`
vs `--patch fused_conv`:
  "stock"   the reference's unpatched fast path (modeling_ipttcdv9.py:
            682-781): two windowed attention calls (this package's band
            kernel), two o_proj GEMMs and two norms, the conv as torch's
            depthwise conv1d behind the reference's rearranges;
  "patched" what patch_fused_attn + patch_triton_conv install: the one-pass
            dual-window kernel (or the LSE variant, kernel="fa3_lse") and the
            conv kernel, the rest as stock;
  "fused"   (default) patched, plus this build's fused epilogue (one o_proj
            GEMM over both outputs, one dual norm) and fused TTT feature pass.
Everything outside the TTT layers is the same in all three.

Fast path and fallback (`_use_fast_prefill_path`, modeling_ipttcdv9.py:
562-574): forward() takes the reference's padding `attention_mask` (B, T)
and packed `cu_seqlens` (B = 1). With either (a mask with a zero), or with
IPTTCD_DISABLE_FAST_PREFILL=1, the TTT layers take the reference's fallback
(:794-850): the teacher and student as two windowed calls, two o_proj GEMMs
and two norms. With a mask or cu_seqlens every layer's attention runs within
each row's unpadded tokens / each packed sequence (fla Attention's varlen
path, fla/layers/attn.py:226-262, on this package's varlen kernel), rotary
positions restart per packed sequence, and the TTT student attends over the
whole rows as the reference's flash_attn_func call does (:825-827).

The output gate (use_output_gate, fla/layers/attn.py:149-167, 284-292) is
applied to both attention outputs on every path, including the patched one,
where the reference's patch drops it (a strict xfail,
test/test_fused_dual_attn.py:339-360).

Prefill onto a populated cache (`cache=IPTTCDv9Cache()`, forward called once
per prompt chunk): each layer keeps the last window_size rotated keys and
values of the tokens already prefilled (all of them for a full-causal model),
fla's window-trimmed attn_state (fla/models/utils.py:35-96), and the next
chunk's queries attend over those keys followed by their own, bottom-right
aligned, through the kernels' Tq < Tk forms (the teacher and, on TTT layers,
the student window; the reference's unpatched fast path does the same with
flash_attn_func on the cached k / v, modeling_ipttcdv9.py:741-751, and its
patched forward falls back to it, profiling/patches.py:270-284). Rotary
positions continue from the tokens already seen. The TTT MLP sees the chunk's
tokens only, as the reference's MLP does. Two deliberate departures, both so
that a chunked prefill attends exactly as one prefill of the whole prompt:
fla's cache rolls a full cache by the chunk length (the first queries of a
later chunk then see fewer than window_size keys); here the kept keys always
reach window_size back from the chunk's first token. And fla's FLACache counts
the chunk's tokens at layer 0, so layers 1.. read a rotary offset one chunk
too far (fla/models/utils.py:326-327, 349-352); here every layer uses the
tokens seen before the chunk.

Not covered (raise NotImplementedError): qkv_bias, non-causal TTT conv,
ttt_weight_renorm, Muon, normalised TTT features or proj-diff,
ttt_output_use_teacher_conv, l2 softmax, a cache together with a padding
mask or packed sequences.
"""
from __future__ import annotations

import os

import torch
import torch.nn.functional as F

from . import attn as _attn
from . import epilogue as _epi
from . import prologue as _pro
from . import ttt as _ttt

# configs/ipttcd/ipttcdv9_qwen3_0.6B_ct_64k_v2_swa8k.json (the config-5 model)
QWEN3_06B_SWA8K = {
    "hidden_size": 1024, "num_hidden_layers": 28, "num_heads": 16, "num_kv_heads": 8,
    "head_dim": 128, "intermediate_size": 3072, "vocab_size": 151936,
    "max_position_embeddings": 65536, "rope_theta": 1000000.0, "window_size": 8192,
    "norm_eps": 1e-06, "initializer_range": 0.02, "tie_word_embeddings": True,
    "qkv_bias": False, "qk_norm": True, "fuse_norm": True, "fuse_swiglu": True,
    "ttt_mode": True, "ttt_layers": [0, 7, 14, 21], "ttt_chunk": 4096, "ttt_lr": 0.3,
    "ttt_proj": True, "ttt_proj_init": "diagonal_gaussian", "ttt_norm_proj_diff": False,
    "ttt_normalize_student_features": False, "ttt_conv": True, "ttt_teacher_conv": True,
    "ttt_student_conv": True, "ttt_teacher_conv_init": "identity",
    "ttt_student_conv_init": "zero", "ttt_output_use_teacher_conv": False,
    "ttt_conv_kernel_size": 5, "ttt_conv_causal": True, "dynamic_lr": True,
    "ttt_visible_chunks": 1, "ttt_update_every": 16, "ttt_weight_renorm": False,
    "use_muon": False,
}

# the reference config classes' defaults for keys a config file may omit
# (configuration_ipttcd.py:16-65, configuration_ipttcdv8.py:12-19,
# configuration_ipttcdv9.py:12-17)
_DEFAULTS = {
    "num_kv_heads": None, "head_dim": None, "qkv_bias": False, "qk_norm": False,
    "window_size": None, "rope_theta": 10000.0, "max_position_embeddings": 2048,
    "hidden_ratio": 4, "intermediate_size": None, "norm_eps": 1e-6,
    "initializer_range": 0.02, "tie_word_embeddings": False, "use_output_gate": False,
    "ttt_mode": False, "ttt_layers": None, "ttt_chunk": 8192, "ttt_lr": 0.3, "ttt_proj": True,
    "ttt_proj_init": "diagonal", "ttt_conv": False, "ttt_teacher_conv": True,
    "ttt_student_conv": True, "ttt_conv_kernel_size": 5, "ttt_conv_causal": True,
    "ttt_teacher_conv_init": "zero", "ttt_student_conv_init": "zero",
    "ttt_output_use_teacher_conv": True, "ttt_output_source": "teacher", "dynamic_lr": True,
    "ttt_visible_chunks": 1, "use_muon": False, "ttt_weight_renorm": False,
    "ttt_norm_proj_diff": False, "ttt_normalize_student_features": True,
    "ttt_update_every": 4, "ttt_fuse_proj_into_update": True, "fuse_norm": True,
    "ttt_scan_state_dtype": "compute", "gate_fn": "sigmoid", "elementwise_affine": True,
    "use_l2_softmax": False,
}


def resolve_config(cfg: dict) -> dict:
    """The reference config with its defaults filled in and the derived sizes
    (num_kv_heads, head_dim, intermediate_size) computed as the reference's
    modules do (fla/layers/attn.py; modeling_ipttcdv9.py:98-102)."""
    c = dict(_DEFAULTS)
    c.update(cfg)
    c["num_kv_heads"] = c["num_kv_heads"] or c["num_heads"]
    c["head_dim"] = c["head_dim"] or c["hidden_size"] // c["num_heads"]
    if c["intermediate_size"] is None:
        inter = int(c["hidden_size"] * c["hidden_ratio"] * 2 / 3)
        c["intermediate_size"] = 256 * ((inter + 256 - 1) // 256)
    c["ttt_layers"] = list(c["ttt_layers"] or []) if c["ttt_mode"] else []
    # the MLP reads ttt_teacher_conv / ttt_student_conv directly; ttt_conv is
    # only their OR (configuration_ipttcdv8.py:32-34, modeling_ipttcdv9.py:130-150)
    c["ttt_teacher_conv"] = bool(c["ttt_teacher_conv"])
    c["ttt_student_conv"] = bool(c["ttt_student_conv"])
    unsupported = [k for k, bad in (
        ("qkv_bias", c["qkv_bias"]), ("use_l2_softmax", c["use_l2_softmax"]),
        ("gate_fn", c["use_output_gate"] and c["gate_fn"] not in ("sigmoid", "swish", "silu")),
        ("ttt_conv_causal=False", c["ttt_layers"] and not c["ttt_conv_causal"]),
        ("ttt_weight_renorm", c["ttt_weight_renorm"]), ("use_muon", c["use_muon"]),
        ("ttt_normalize_student_features", c["ttt_layers"] and c["ttt_normalize_student_features"]),
        ("ttt_norm_proj_diff", c["ttt_norm_proj_diff"]),
        ("ttt_output_use_teacher_conv", c["ttt_layers"] and c["ttt_output_use_teacher_conv"]),
        ("ttt_output_source", c["ttt_output_source"] != "teacher"),
        ("ttt_fuse_proj_into_update=False", not c["ttt_fuse_proj_into_update"]),
        # nn.RMSNorm with a rounded residual add (configuration_ipttcd.py:37, 89)
        ("fuse_norm=False", not c["fuse_norm"]),
        # an fp32 or bf16 scan state instead of the compute dtype
        # (configuration_ipttcdv9.py:17-34, modeling_ipttcdv9.py:180-181)
        ("ttt_scan_state_dtype", str(c["ttt_scan_state_dtype"]).lower() != "compute"),
    ) if bad]
    if unsupported:
        raise NotImplementedError(f"ipttcdv9 prefill: unsupported options {unsupported}")
    if c["use_output_gate"] and c["num_kv_heads"] != c["num_heads"]:
        # fla's g_proj has kv_dim outputs (fla/layers/attn.py:151): the gate
        # multiplies the (num_heads * head_dim) output only when they match
        raise ValueError("use_output_gate needs num_kv_heads == num_heads (g_proj outputs "
                         "num_kv_heads * head_dim, the attention output num_heads * head_dim)")
    return c


def _fused_gate(c: dict) -> bool:
    """FusedRMSNormGated (swish gate with fuse_norm, fla/layers/attn.py:152-158)."""
    return c["gate_fn"] == "swish" and c["fuse_norm"]


def init_weights(cfg: dict, device, dtype=torch.bfloat16, seed: int = 0) -> dict:
    """Random parameters with the reference's initialisation
    (modeling_ipttcdv9.py:885-996 over fla's TransformerPreTrainedModel
    init): Linear and Embedding N(0, initializer_range); norms ones; ttt_proj
    per ttt_proj_init; TTT convs per ttt_{teacher,student}_conv_init; b_proj
    N(0, initializer_range). Drawn in fp32 on `device` from `seed`, then cast
    to `dtype` (as build_model casts the fp32 model, bench_prefill.py:76-77)."""
    c = resolve_config(cfg)
    g = torch.Generator(device=device).manual_seed(seed)
    std = c["initializer_range"]
    H, I, D = c["hidden_size"], c["intermediate_size"], c["head_dim"]
    Hq, Hkv, K = c["num_heads"], c["num_kv_heads"], c["ttt_conv_kernel_size"]

    def normal(*shape):
        return (torch.randn(*shape, generator=g, device=device) * std).to(dtype)

    def ones(n):
        return torch.ones(n, device=device, dtype=dtype)

    w = {"model.embeddings.weight": normal(c["vocab_size"], H)}
    for i in range(c["num_hidden_layers"]):
        p = f"model.layers.{i}."
        w[p + "attn_norm.weight"] = ones(H)
        w[p + "attn.q_proj.weight"] = normal(Hq * D, H)
        w[p + "attn.k_proj.weight"] = normal(Hkv * D, H)
        w[p + "attn.v_proj.weight"] = normal(Hkv * D, H)
        w[p + "attn.o_proj.weight"] = normal(H, Hq * D)
        if c["qk_norm"]:
            w[p + "attn.q_norm.weight"] = ones(D)
            w[p + "attn.k_norm.weight"] = ones(D)
        if c["use_output_gate"]:
            w[p + "attn.g_proj.weight"] = normal(Hkv * D, H)
            if c["elementwise_affine"]:
                gname = "g_norm_swish_gate" if _fused_gate(c) else "g_norm"
                w[p + f"attn.{gname}.weight"] = ones(D)
        w[p + "mlp_norm.weight"] = ones(H)
        w[p + "mlp.gate_proj.weight"] = normal(I, H)
        w[p + "mlp.up_proj.weight"] = normal(I, H)
        w[p + "mlp.down_proj.weight"] = normal(H, I)
        if i in c["ttt_layers"]:
            if c["ttt_proj"]:
                init = c["ttt_proj_init"]
                if init == "diagonal":
                    pw = torch.eye(H, device=device) * std
                elif init == "diagonal_gaussian":
                    pw = torch.diag(torch.randn(H, generator=g, device=device) * std)
                elif init == "zero":
                    pw = torch.zeros(H, H, device=device)
                else:
                    pw = torch.randn(H, H, generator=g, device=device) * std
                w[p + "mlp.ttt_proj.weight"] = pw.to(dtype)
            for role in ("teacher", "student"):
                if not c[f"ttt_{role}_conv"]:
                    continue
                init = c[f"ttt_{role}_conv_init"]
                cw = torch.zeros(I, 1, K, device=device)
                if init == "identity":
                    cw[:, 0, K - 1] = 1.0  # causal conv: the last tap is the current position
                elif init == "random":
                    cw = torch.randn(I, 1, K, generator=g, device=device) * std
                w[p + f"mlp.ttt_{role}_conv.weight"] = cw.to(dtype)
            if c["dynamic_lr"]:
                w[p + "mlp.b_proj"] = normal(H)
    w["model.norm.weight"] = ones(H)
    w["lm_head.weight"] = (w["model.embeddings.weight"] if c["tie_word_embeddings"]
                           else normal(c["vocab_size"], H))
    return w


PATHS = ("stock", "patched", "fused")


class IPTTCDv9Prefill:
    """Prefill-only ipttcdv9 on one GPU. `weights` uses the reference's
    state-dict names (e.g. from init_weights, or a safetensors checkpoint of the
    reference model cast to bf16). `path` selects the TTT layers' path
    ("stock", "patched" or "fused")."""

    def __init__(self, cfg: dict, weights: dict, path: str = "fused"):
        if path not in PATHS:
            raise ValueError(f"path must be one of {PATHS}, got {path!r}")
        self.attn_kernel = "two_calls" if path == "stock" else "triton"
        self.conv_kernel = path != "stock"
        self.fuse_extra = path == "fused"
        self.cfg = c = resolve_config(cfg)
        self.w = weights
        self.dev = weights["model.embeddings.weight"].device
        self.dtype = weights["model.embeddings.weight"].dtype
        H, D = c["hidden_size"], c["head_dim"]
        self.Hq, self.Hkv, self.D = c["num_heads"], c["num_kv_heads"], D
        # stacked projection weights: one GEMM for q|k|v, one for gate|up
        self.qkv_w, self.gu_w, self.ttt = [], [], {}
        for i in range(c["num_hidden_layers"]):
            p = f"model.layers.{i}."
            self.qkv_w.append(torch.cat([weights[p + "attn.q_proj.weight"],
                                         weights[p + "attn.k_proj.weight"],
                                         weights[p + "attn.v_proj.weight"]], 0).contiguous())
            self.gu_w.append(torch.cat([weights[p + "mlp.gate_proj.weight"],
                                        weights[p + "mlp.up_proj.weight"]], 0).contiguous())
            if i in c["ttt_layers"]:
                self.ttt[i] = _ttt.TttMlpWeights(
                    self.gu_w[i], weights[p + "mlp.down_proj.weight"],
                    weights.get(p + "mlp.ttt_proj.weight"),
                    weights.get(p + "mlp.ttt_teacher_conv.weight"),
                    weights.get(p + "mlp.ttt_student_conv.weight"),
                    weights.get(p + "mlp.b_proj"))
        # rotary tables of the reference's cache length (max_seqlen is at least
        # max_position_embeddings, fla/layers/attn.py:200-213), from fp32 inv_freq
        self._inv_freq = _pro.rope_inv_freq(D, c["rope_theta"], self.dev)
        self._tables = None
        self.window_t = c["window_size"] if c["window_size"] is not None else -1
        self.window_s = c["ttt_visible_chunks"] * c["ttt_chunk"]

    def tables(self, T: int):
        """Rotary cos / sin tables of at least T rows (the reference's cache
        length, extended when a cached prefill reaches past it)."""
        rows = max(T, self.cfg["max_position_embeddings"] or 0)
        if self._tables is None or self._tables[0].shape[0] < rows:
            self._tables = _pro.rope_tables(self._inv_freq, rows, self.dtype)
        return self._tables

    # ------------------------------------------------------------------ layers

    def _qkv(self, i: int, x: torch.Tensor, ctx: "_Prefill"):
        c, w = self.cfg, self.w
        B, T, _ = x.shape
        Hq, Hkv, D = self.Hq, self.Hkv, self.D
        qkv = F.linear(x, self.qkv_w[i])
        q = qkv[..., :Hq * D].view(B, T, Hq, D)
        k = qkv[..., Hq * D:(Hq + Hkv) * D].view(B, T, Hkv, D)
        v = qkv[..., (Hq + Hkv) * D:].view(B, T, Hkv, D)
        p = f"model.layers.{i}.attn."
        cos, sin = ctx.tables if ctx.tables is not None else self.tables(ctx.offset + T)
        qw = w.get(p + "q_norm.weight") if c["qk_norm"] else None
        kw = w.get(p + "k_norm.weight") if c["qk_norm"] else None
        # fla's RMSNorm default eps for q_norm / k_norm (fla/layers/attn.py:61-63)
        q, k = _pro.qk_norm_rope(q, k, qw, kw, 1e-5, cos, sin, ctx.offset)
        return q, k, v

    @property
    def path(self) -> str:
        if self.attn_kernel == "two_calls" and not self.conv_kernel:
            return "stock"
        return "fused" if self.fuse_extra else "patched"

    def _teacher_attention(self, q, k, v, ctx: "_Prefill"):
        """The teacher window within each row's unpadded tokens / each packed
        sequence (fla Attention's varlen path) or over whole rows."""
        if ctx.cu_seqlens is None:
            return _attn.window_attn(q, k, v, self.window_t)
        B, T, Hq, D = q.shape
        W = self.window_t if self.window_t >= 0 else ctx.max_seqlen
        if ctx.indices is None:  # packed sequences, B = 1
            o = _attn.band_attn_varlen(q[0], k[0], v[0], ctx.cu_seqlens, ctx.max_seqlen, 0, W)
            return o.view(B, T, Hq, D)
        idx = ctx.indices
        o = torch.zeros(B * T, Hq, D, dtype=q.dtype, device=q.device)
        o[idx] = _attn.band_attn_varlen(
            q.reshape(B * T, Hq, D)[idx], k.reshape(B * T, -1, D)[idx],
            v.reshape(B * T, -1, D)[idx], ctx.cu_seqlens, ctx.max_seqlen, 0, W)
        return o.view(B, T, Hq, D)

    def _gate(self, i: int, x: torch.Tensor, o: torch.Tensor) -> torch.Tensor:
        """The attention output gate (fla/layers/attn.py:284-292) on o
        (B, T, H, D) with x the attn_norm output; returns (B, T, H*D)."""
        B, T = o.shape[0], o.shape[1]
        if not self.cfg["use_output_gate"]:
            return o.reshape(B, T, -1)
        c, w = self.cfg, self.w
        p = f"model.layers.{i}.attn."
        D = self.D
        g = F.linear(x, w[p + "g_proj.weight"])
        if _fused_gate(c):
            # FusedRMSNormGated: rmsnorm(o) * w * g * sigmoid(g) in fp32, one
            # rounding (fla/modules/fused_norm_gate.py:91-95)
            of = o.float()
            y = of * torch.rsqrt(of.pow(2).mean(-1, keepdim=True) + c["norm_eps"])
            nw = w.get(p + "g_norm_swish_gate.weight")
            if nw is not None:
                y = y * nw.float()
            gf = g.float().view(B, T, -1, D)
            return (y * gf * torch.sigmoid(gf)).to(o.dtype).reshape(B, T, -1)
        nw = w.get(p + "g_norm.weight")
        if nw is None:
            nw = torch.ones(D, dtype=o.dtype, device=o.device)
        on = _epi.rmsnorm(o.reshape(-1, D).contiguous(), nw, c["norm_eps"]).view(B, T, -1)
        act = torch.sigmoid(g) if c["gate_fn"] == "sigmoid" else F.silu(g)
        return on * act

    def _ttt_attention(self, q, k, v):
        """Teacher and student outputs of a TTT layer; k / v may be longer than q
        (a cached prefill: the queries are the last positions)."""
        if self.attn_kernel == "triton":
            return _attn.fused_dual_window_attn(q, k, v, self.window_t, self.window_s)
        if self.attn_kernel == "fa3_lse":
            return _attn.lse_dual_window_attn_fa3_fast(q, k, v, self.window_t, self.window_s)
        return (_attn.window_attn(q, k, v, self.window_t),
                _attn.window_attn(q, k, v, self.window_s))

    def layer(self, i: int, h: torch.Tensor, y_prev: torch.Tensor | None = None,
              ctx: "_Prefill | None" = None):
        """One block. With y_prev, the block input is h + y_prev (the previous
        block's closing residual add), fused with this block's attn_norm.
        Returns (residual, y): the block output is residual + y."""
        c, w = self.cfg, self.w
        p = f"model.layers.{i}."
        eps = c["norm_eps"]
        B, T, H = h.shape
        ctx = ctx if ctx is not None else _Prefill()
        if y_prev is None:
            residual = h
            x = _epi.rmsnorm(h, w[p + "attn_norm.weight"], eps)
        else:
            x, residual = _epi.add_rmsnorm(y_prev, h, w[p + "attn_norm.weight"], eps)
        xa = x  # attn_norm output: the gate's input
        q, k, v = self._qkv(i, x, ctx)
        if ctx.cache is not None:
            # the cached keys of earlier chunks, then this chunk's (Tk >= T)
            k, v = ctx.cache.extend(i, k, v, None if self.window_t < 0 else self.window_t)
        o_w = w[p + "attn.o_proj.weight"]
        gated = c["use_output_gate"]
        if i in self.ttt and T >= c["ttt_chunk"]:
            norm = _NormView(w[p + "mlp_norm.weight"], eps)
            proj = _LinearView(o_w)
            if ctx.fast:
                o_t, o_s = self._ttt_attention(q, k, v)
            else:
                # the reference's fallback (modeling_ipttcdv9.py:794-850): the
                # teacher through the (unpad-aware) attention, the student a
                # windowed call on the whole rows
                o_t = self._teacher_attention(q, k, v, ctx)
                o_s = _attn.window_attn(q, k, v, self.window_s)
            if gated:
                o_t, o_s = self._gate(i, xa, o_t), self._gate(i, xa, o_s)
            if self.fuse_extra and ctx.fast:
                x, residual, s = _epi.fused_attn_epilogue(proj, norm, o_t, o_s, residual)
            else:
                a_t = F.linear(o_t.reshape(B, T, -1), o_w)
                a_s = F.linear(o_s.reshape(B, T, -1), o_w)
                s, _ = _epi.rmsnorm(a_s, w[p + "mlp_norm.weight"], eps, residual=residual)
                x, residual = _epi.rmsnorm(a_t, w[p + "mlp_norm.weight"], eps, residual=residual)
            y = _ttt.ttt_mlp(x, s, self.ttt[i], chunk=c["ttt_chunk"], lr=c["ttt_lr"],
                             update_every=c["ttt_update_every"], fused=self.fuse_extra,
                             conv="kernel" if self.conv_kernel else "stock",
                             scan="kernel" if self.fuse_extra else "torch")
        else:
            o = self._teacher_attention(q, k, v, ctx)
            a = F.linear(self._gate(i, xa, o), o_w)
            x, residual = _epi.rmsnorm(a, w[p + "mlp_norm.weight"], eps, residual=residual)
            y = _ttt.swiglu_mlp(x, self.gu_w[i], w[p + "mlp.down_proj.weight"])
        return residual, y

    def _prefill_context(self, B: int, T: int, attention_mask, cu_seqlens,
                         cache: "IPTTCDv9Cache | None" = None) -> "_Prefill":
        """_use_fast_prefill_path (modeling_ipttcdv9.py:562-574) and what the
        fallback needs: unpad indices and cu_seqlens for a padding mask,
        per-sequence rotary tables for packed sequences; the rotary offset and
        the cache of a cached prefill."""
        ctx = _Prefill()
        if cache is not None:
            if not isinstance(cache, IPTTCDv9Cache):
                raise ValueError("cache must be an IPTTCDv9Cache")
            if cu_seqlens is not None or (attention_mask is not None
                                          and not bool(attention_mask.to(self.dev).bool().all())):
                raise NotImplementedError("a cached prefill with a padding mask or packed "
                                          "sequences")
            cache.check(B, self.Hkv, self.D, self.dtype, self.dev)
            ctx.cache, ctx.offset = cache, cache.seen
            attention_mask = None
        if attention_mask is not None:
            if attention_mask.shape != (B, T):
                raise ValueError(f"attention_mask must be (B, T) = ({B}, {T}), got "
                                 f"{tuple(attention_mask.shape)}")
            m = attention_mask.to(self.dev).bool()
            if not bool(m.all()):  # a host sync, as the reference's gate makes
                if cu_seqlens is not None:
                    raise ValueError("pass either a padding attention_mask or cu_seqlens")
                lens = m.sum(1, dtype=torch.int32)
                ctx.indices = m.reshape(-1).nonzero().flatten()
                ctx.cu_seqlens = F.pad(torch.cumsum(lens, 0, dtype=torch.int32), (1, 0))
                ctx.max_seqlen = int(lens.max().item())
        if cu_seqlens is not None:
            if B != 1:
                raise ValueError("cu_seqlens needs a packed batch of one row (B = 1)")
            cu = torch.as_tensor(cu_seqlens, dtype=torch.int32, device=self.dev)
            cu_h = cu.cpu()
            if cu_h[0] != 0 or int(cu_h[-1]) != T or bool((cu_h[1:] < cu_h[:-1]).any()):
                raise ValueError("cu_seqlens must rise from 0 to T")
            ctx.cu_seqlens = cu
            ctx.max_seqlen = int((cu_h[1:] - cu_h[:-1]).max().item())
            # rotary positions restart at every sequence (fla's varlen rotary)
            seq = torch.repeat_interleave(torch.arange(cu_h.numel() - 1, device=self.dev),
                                          (cu[1:] - cu[:-1]).long())
            pos = torch.arange(T, device=self.dev) - cu[:-1].long()[seq]
            cos, sin = self.tables(T)
            ctx.tables = (cos[pos].contiguous(), sin[pos].contiguous())
        ctx.fast = (os.environ.get("IPTTCD_DISABLE_FAST_PREFILL") != "1"
                    and ctx.cu_seqlens is None)
        return ctx

    @torch.inference_mode()
    def forward(self, input_ids: torch.Tensor, logits_to_keep: int = 1,
                attention_mask: torch.Tensor | None = None,
                cu_seqlens: torch.Tensor | None = None,
                cache: "IPTTCDv9Cache | None" = None) -> torch.Tensor:
        """Logits (B, logits_to_keep, vocab) of the prefill of `input_ids`
        (B, T), as IPTTCDForCausalLM(input_ids, logits_to_keep=...) returns them
        with fuse_linear_cross_entropy off (bench_prefill.py:73-74).
        attention_mask: the (B, T) 0/1 padding mask; cu_seqlens: packed
        sequences of a (1, T) batch (int32, 0 .. T); cache: an IPTTCDv9Cache
        holding the earlier chunks of the prompt (empty for the first), which
        this call extends with its T tokens."""
        if input_ids.dim() != 2 or input_ids.device != self.dev:
            raise ValueError("input_ids must be (B, T) on the model's device")
        B, T = input_ids.shape
        ctx = self._prefill_context(B, T, attention_mask, cu_seqlens, cache)
        h = F.embedding(input_ids, self.w["model.embeddings.weight"])
        y = None
        for i in range(self.cfg["num_hidden_layers"]):
            h, y = self.layer(i, h, y, ctx)
        if cache is not None:
            cache.seen += T
        if logits_to_keep > 0:  # only the kept rows of the last block's output
            h, y = h[:, -logits_to_keep:], y[:, -logits_to_keep:]
        keep = h + y
        x = _epi.rmsnorm(keep.contiguous(), self.w["model.norm.weight"], self.cfg["norm_eps"])
        return F.linear(x, self.w["lm_head.weight"])


def patch_fused_attn(model: IPTTCDv9Prefill, kernel: str = "triton") -> int:
    """profiling/patches.py:215-312 on this model: the TTT layers' two windowed
    calls become the one-pass dual-window kernel ("triton", the reference's
    name for it) or the LSE-combination variant ("fa3_lse"). Returns the
    number of TTT layers patched, as the reference's hook does."""
    if kernel not in ("triton", "fa3_lse"):
        raise ValueError(kernel)
    model.attn_kernel = kernel
    return len(model.ttt)


def patch_triton_conv(model: IPTTCDv9Prefill) -> int:
    """profiling/patches.py:411-432 on this model: the TTT convs run on the
    chunk-local conv kernel instead of the rearranged torch conv."""
    model.conv_kernel = True
    return len(model.ttt)


class IPTTCDv9Cache:
    """The K/V cache of a prefill in chunks: per layer the rotated keys and the
    values of the last `window_size` tokens already prefilled (all of them
    when the model attends full-causally), fla's window-trimmed attn_state
    (fla/models/utils.py:35-96), and the count of tokens seen. Pass the same
    object to every IPTTCDv9Prefill.forward of one prompt."""

    def __init__(self):
        self.seen = 0
        self.kv: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
        self._shape = None

    def check(self, B: int, Hkv: int, D: int, dtype, device) -> None:
        shape = (B, Hkv, D, dtype, torch.device(device))
        if self._shape is not None and self._shape != shape:
            raise ValueError(f"cache holds (B, Hkv, D, dtype, device) = {self._shape}, "
                             f"this prefill needs {shape}")
        self._shape = shape

    def extend(self, layer: int, k: torch.Tensor, v: torch.Tensor, keep: int | None):
        """Keys / values for layer's attention: the cached ones, then k / v of
        this chunk (B, T, Hkv, D). Keeps the last `keep` of them (all with None)
        for the next chunk."""
        old = self.kv.get(layer)
        if old is not None:
            k = torch.cat([old[0], k], 1)
            v = torch.cat([old[1], v], 1)
        n = k.shape[1] if keep is None else min(keep, k.shape[1])
        self.kv[layer] = (k[:, k.shape[1] - n:].contiguous(), v[:, v.shape[1] - n:].contiguous())
        return k, v


class _Prefill:
    """Per-forward state of the fast-path gate and the fallback."""

    def __init__(self):
        self.fast = True          # _use_fast_prefill_path
        self.indices = None       # unpadded token rows of a padded batch
        self.cu_seqlens = None    # int32 sequence starts (unpadded rows or packed)
        self.max_seqlen = 0
        self.tables = None        # per-token rotary rows for packed sequences
        self.cache = None         # IPTTCDv9Cache of a cached prefill
        self.offset = 0           # rotary offset: tokens prefilled before this call


class _NormView:
    """The attributes of an fla RMSNorm module that fused_attn_epilogue reads."""

    def __init__(self, weight, eps):
        self.weight, self.bias, self.eps = weight, None, eps


class _LinearView:
    def __init__(self, weight):
        self.weight, self.bias = weight, None


def prefill_flops(cfg: dict, B: int, T: int) -> dict:
    """Algorithmic FLOPs of one prefill by part (GEMMs 2*m*n*k; attention
    4*Hq*D per in-band pair, the teacher band once on TTT layers)."""
    from math import ceil
    c = resolve_config(cfg)
    H, I, D = c["hidden_size"], c["intermediate_size"], c["head_dim"]
    Hq, Hkv, L = c["num_heads"], c["num_kv_heads"], c["num_hidden_layers"]
    n_ttt = sum(1 for i in c["ttt_layers"] if i < L)
    W = c["window_size"]

    def pairs(W):
        if W is None or W >= T:
            return T * (T + 1) // 2
        return W * (W + 1) // 2 + (T - W) * W

    tok = B * T
    proj = 2 * tok * H * (Hq + 2 * Hkv) * D + 2 * tok * Hq * D * H
    mlp = 2 * tok * H * 2 * I + 2 * tok * I * H
    attn = 4 * B * Hq * D * pairs(W)
    C = c["ttt_chunk"]
    nch = ceil(T / C)
    ttt_extra = (2 * tok * Hq * D * H            # student o_proj
                 + 2 * tok * H * 2 * I           # student gate|up
                 + 2 * B * (nch - 1) * C * I * H  # diff @ W_update
                 + 2 * B * (nch - 1) * H * C * I  # dW
                 + 2 * I * H * H)                # W_update = W_down^T @ P
    return {"gemm": L * (proj + mlp) + n_ttt * ttt_extra, "attention": L * attn,
            "lm_head": 2 * B * H * c["vocab_size"]}
