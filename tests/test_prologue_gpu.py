"""Attention prologue on the GPU (through the C ABI): the fused q/k RMSNorm +
rotary kernel and the rotary-table kernel against the CPU oracle, on the
same inputs and tables."""
from __future__ import annotations

import types

import pytest
import torch

from conftest import random_cases

from oracle import attn_ref, prologue_ref
from ttcd_amd import prologue

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rand(shape, dtype=torch.bfloat16, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _weights(D, dtype, seed):
    # around 1, as a trained qk_norm weight
    return (1.0 + 0.2 * _rand((D,), torch.float32, seed)).to(dtype)


CASES = [
    # B, T, Hq, Hkv, D, norm, dtype, w_dtype, offset, base
    pytest.param(2, 257, 16, 8, 128, True, torch.bfloat16, torch.bfloat16, 0, 1e6, id="qwen3-bf16"),
    pytest.param(1, 300, 16, 8, 128, True, torch.bfloat16, torch.float32, 1000, 1e6, id="offset-f32w"),
    pytest.param(1, 131, 15, 5, 64, False, torch.bfloat16, None, 0, 1e5, id="smollm2-rope-only"),
    pytest.param(2, 77, 4, 1, 64, True, torch.float16, torch.float16, 3, 1e4, id="f16-mqa"),
    pytest.param(1, 1, 3, 3, 128, True, torch.bfloat16, torch.bfloat16, 0, 1e6, id="one-token"),
    pytest.param(1, 64, 16, 8, 128, True, torch.bfloat16, torch.bfloat16, 65536 - 64, 1e6,
                 id="last-positions"),
]


def _check_two_stages(q, k, wq, wk, eps, cos, sin, offset, qo, ko):
    """The norm stage within one rounding of the oracle, and the rotation of
    the kernel's own normed values bit for bit (every rotated output is one
    correctly rounded value of its inputs). A direct ulp bound on the fused
    output would be loose: where x0*c - x1*s cancels, one ulp of the normed
    input is several ulps of the output."""
    dev = qo.device
    R = q.shape[-1] // 2
    T = q.shape[1]
    ones = torch.ones(offset + T, R, dtype=q.dtype, device=dev)
    zeros = torch.zeros(offset + T, R, dtype=q.dtype, device=dev)
    with torch.inference_mode():
        nq, nk = prologue.qk_norm_rope(q.to(dev), k.to(dev), wq.to(dev), wk.to(dev), eps, ones,
                                       zeros, offset)
    torch.cuda.synchronize()
    for n, x, w in ((nq, q, wq), (nk, k, wk)):
        rep = attn_ref.ulp_report(n.cpu(), prologue_ref.rms_norm_ref(x.cpu(), w.cpu(), eps))
        assert rep["max_ulp"] <= 1 and rep["bit_equal_pct"] > 99.0, rep
    for got, n in ((qo, nq), (ko, nk)):
        assert torch.equal(got.cpu(), prologue_ref.rope_ref(n.cpu(), cos.cpu(), sin.cpu(), offset))


@pytest.mark.parametrize("B,T,Hq,Hkv,D,norm,dtype,wdt,offset,base", CASES)
def test_matches_oracle(B, T, Hq, Hkv, D, norm, dtype, wdt, offset, base):
    q = _rand((B, T, Hq, D), dtype, 1, 2.0)
    k = _rand((B, T, Hkv, D), dtype, 2, 2.0)
    wq = _weights(D, wdt, 3) if norm else None
    wk = _weights(D, wdt, 4) if norm else None
    inv = prologue.rope_inv_freq(D, base, DEV)
    cos, sin = prologue.rope_tables(inv, offset + T, dtype)
    with torch.inference_mode():
        qo, ko = prologue.qk_norm_rope(q.to(DEV), k.to(DEV), wq.to(DEV) if norm else None,
                                       wk.to(DEV) if norm else None, 1e-5, cos, sin, offset)
    torch.cuda.synchronize()
    if not norm:
        # rotation only: every output is one correctly rounded value
        rq, rk = prologue_ref.qk_norm_rope_ref(q, k, None, None, 0.0, cos.cpu(), sin.cpu(),
                                               offset)
        assert torch.equal(qo.cpu(), rq) and torch.equal(ko.cpu(), rk)
    else:
        _check_two_stages(q, k, wq, wk, 1e-5, cos, sin, offset, qo, ko)


def test_tables_match_oracle_and_torch():
    # the reference builds its tables with torch on the model's GPU
    # (fla/modules/rotary.py:464-486); ours must agree with that and with
    # float64 cos / sin of the same fp32 products
    D, rows = 128, 65536
    inv = prologue.rope_inv_freq(D, 1e6, DEV)
    cos, sin = prologue.rope_tables(inv, rows, torch.bfloat16)
    t = torch.arange(rows, device=DEV, dtype=torch.float32)
    freqs = torch.outer(t, inv)
    tc, ts = torch.cos(freqs).to(torch.bfloat16), torch.sin(freqs).to(torch.bfloat16)
    torch.cuda.synchronize()
    for got, want in ((cos, tc), (sin, ts)):
        rep = attn_ref.ulp_report(got.cpu(), want.cpu())
        assert rep["max_ulp"] <= 1 and rep["bit_equal_pct"] > 99.99, rep
    oc, os_ = prologue_ref.tables_ref(inv.cpu(), rows)
    for got, want in ((cos, oc), (sin, os_)):
        rep = attn_ref.ulp_report(got.cpu(), want)
        assert rep["max_ulp"] <= 1 and rep["bit_equal_pct"] > 99.9, rep


def test_strided_inputs_from_a_fused_projection():
    # q and k as views of one (B, T, (Hq + 2 Hkv) * D) projection output
    B, T, Hq, Hkv, D = 2, 96, 8, 2, 128
    qkv = _rand((B, T, (Hq + 2 * Hkv) * D), seed=5).to(DEV)
    q = qkv[..., :Hq * D].view(B, T, Hq, D)
    k = qkv[..., Hq * D:(Hq + Hkv) * D].view(B, T, Hkv, D)
    w = _weights(D, torch.bfloat16, 6).to(DEV)
    cos, sin = prologue.rope_tables(prologue.rope_inv_freq(D, 1e6, DEV), T)
    with torch.inference_mode():
        a = prologue.qk_norm_rope(q, k, w, w, 1e-6, cos, sin)
        b = prologue.qk_norm_rope(q.contiguous(), k.contiguous(), w, w, 1e-6, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_drop_in_on_an_attention_module():
    # the fused call on a stand-in with the fla Attention attributes it reads
    B, T, Hq, Hkv, D = 1, 200, 16, 8, 128
    wq, wk = _weights(D, torch.bfloat16, 7).to(DEV), _weights(D, torch.bfloat16, 8).to(DEV)
    rot = torch.nn.Module()
    rot.register_buffer("inv_freq", prologue.rope_inv_freq(D, 1e6, DEV))
    rot.interleaved, rot.scale, rot._yarn_attn_scaling = False, None, 1.0
    attn = types.SimpleNamespace(
        qk_norm=True, use_nope=False, rotary=rot,
        q_norm=types.SimpleNamespace(weight=wq, bias=None, eps=1e-5),
        k_norm=types.SimpleNamespace(weight=wk, bias=None, eps=1e-5))
    q = _rand((B, T, Hq, D), seed=9).to(DEV)
    k = _rand((B, T, Hkv, D), seed=10).to(DEV)
    with torch.inference_mode():
        fq, fk = prologue.fused_qk_norm_rope(attn, q, k, seqlen_offset=0, max_seqlen=4096)
        cos, sin = prologue.rope_tables(rot.inv_freq, 4096)
        eq, ek = prologue.qk_norm_rope(q, k, wq, wk, 1e-5, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(fq, eq) and torch.equal(fk, ek)
    _check_two_stages(q.cpu(), k.cpu(), wq.cpu(), wk.cpu(), 1e-5, cos, sin, 0, fq, fk)
    # use_nope: norm only, rotation skipped
    attn.use_nope = True
    with torch.inference_mode():
        nq, _ = prologue.fused_qk_norm_rope(attn, q, k)
    torch.cuda.synchronize()
    assert attn_ref.ulp_report(nq.cpu(), prologue_ref.rms_norm_ref(q.cpu(), wq.cpu(),
                                                                    1e-5))["max_ulp"] <= 1


def test_headline_shape_sampled_rows():
    # Qwen3-0.6B layer at 64K: every row of a strided sample against the oracle
    B, T, Hq, Hkv, D = 1, 65536, 16, 8, 128
    g = torch.Generator(device=DEV).manual_seed(0)
    q = torch.randn(B, T, Hq, D, device=DEV, dtype=torch.bfloat16, generator=g)
    k = torch.randn(B, T, Hkv, D, device=DEV, dtype=torch.bfloat16, generator=g)
    w = (1.0 + 0.2 * torch.randn(D, device=DEV, generator=g)).to(torch.bfloat16)
    cos, sin = prologue.rope_tables(prologue.rope_inv_freq(D, 1e6, DEV), T)
    with torch.inference_mode():
        qo, ko = prologue.qk_norm_rope(q, k, w, w, 1e-5, cos, sin)
    torch.cuda.synchronize()
    rows = torch.arange(0, T, 61)
    # the norm stage on the full tensors (identity tables), then both stages
    # on the sampled rows
    ones = torch.ones(T, D // 2, dtype=q.dtype, device=DEV)
    zeros = torch.zeros(T, D // 2, dtype=q.dtype, device=DEV)
    with torch.inference_mode():
        nq, nk = prologue.qk_norm_rope(q, k, w, w, 1e-5, ones, zeros)
    torch.cuda.synchronize()
    for got, n, x in ((qo, nq, q), (ko, nk, k)):
        rep = attn_ref.ulp_report(n[:, rows].cpu(),
                                  prologue_ref.rms_norm_ref(x[:, rows].cpu(), w.cpu(), 1e-5))
        assert rep["max_ulp"] <= 1 and rep["bit_equal_pct"] > 99.0, rep
        assert torch.equal(got[:, rows].cpu(), prologue_ref.rope_ref(
            n[:, rows].cpu(), cos[rows].cpu(), sin[rows].cpu()))


def _random_prologue_case(i):
    import random
    r = random.Random(5000 + i)
    Hkv = r.choice([1, 2, 4, 8])
    return dict(B=r.choice([1, 2]), T=r.randint(1, 700), Hq=Hkv * r.choice([1, 2, 3]), Hkv=Hkv,
                D=r.choice([64, 128]), norm=r.random() < 0.75,
                dtype=r.choice([torch.bfloat16, torch.bfloat16, torch.float16]),
                wdt=r.choice(["x", "x", torch.float32]), offset=r.choice([0, 0, r.randint(1, 70000)]),
                base=r.choice([1e4, 1e5, 1e6]))


@pytest.mark.parametrize("i", range(random_cases(30)))
def test_random_shapes_match_oracle(i):
    """Seeded random batches, lengths, head counts, head dims, dtypes, weight dtypes,
    positions and rotary bases against the oracle, with the bounds of test_matches_oracle."""
    c = _random_prologue_case(i)
    print(f"case {i}: {c}", flush=True)
    wdt = c["dtype"] if c["wdt"] == "x" else c["wdt"]
    test_matches_oracle(c["B"], c["T"], c["Hq"], c["Hkv"], c["D"], c["norm"], c["dtype"], wdt,
                        c["offset"], c["base"])
