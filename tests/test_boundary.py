"""The drop-in boundary as the reference's caller sees it.

profiling/patches.py imports the hot path by bare module name from a directory
on sys.path (patches.py:227 ``from fused_dual_attn import
fused_dual_window_attn``, :229 ``from lse_dual_attn import
lse_dual_window_attn_fa3_fast as fused_dual_window_attn``, :414 ``from
fused_conv import causal_dwconv_chunked``). These tests put
ttcd_amd/profiling first on sys.path in a fresh interpreter, import the
modules exactly that way, and hold their signatures to the reference's:
the reference's parameters in the same order, kinds and defaults, and
anything added keyword-only with a default (so every call patches.py or the
benches make binds the same way). The GPU half calls through the bare-name
modules and requires outputs bit-identical to the ttcd_amd calls.
"""
from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN = os.path.join(REPO, "ttcd_amd", "profiling")

# (name, kind, default) of each parameter, from the reference's definitions.
# "P" = positional-or-keyword; "-" = no default.
REFERENCE_SIGNATURES = {
    # profiling/fused_dual_attn.py:244-246
    ("fused_dual_attn", "fused_dual_window_attn"): [
        ("q", "P", "-"), ("k", "P", "-"), ("v", "P", "-"), ("window_teacher", "P", "-"),
        ("window_student", "P", "-"), ("block_n", "P", "64")],
    # profiling/lse_dual_attn.py:16
    ("lse_dual_attn", "lse_dual_window_attn"): [
        ("q", "P", "-"), ("k", "P", "-"), ("v", "P", "-"), ("window_teacher", "P", "-"),
        ("window_student", "P", "-")],
    # profiling/lse_dual_attn.py:74
    ("lse_dual_attn", "lse_dual_window_attn_fa3"): [
        ("q", "P", "-"), ("k", "P", "-"), ("v", "P", "-"), ("window_teacher", "P", "-"),
        ("window_student", "P", "-")],
    # profiling/lse_dual_attn.py:134
    ("lse_dual_attn", "lse_dual_window_attn_fa3_fast"): [
        ("q", "P", "-"), ("k", "P", "-"), ("v", "P", "-"), ("window_teacher", "P", "-"),
        ("window_student", "P", "-")],
    # profiling/fused_conv.py:51
    ("fused_conv", "causal_dwconv_chunked"): [("x", "P", "-"), ("conv", "P", "-")],
}

_PROBE = r"""
import inspect, json, sys
sys.path.insert(0, sys.argv[1])
out = {}
# the import statements of patches.py:227, :229 and :414, verbatim in form
from fused_dual_attn import fused_dual_window_attn
from lse_dual_attn import lse_dual_window_attn_fa3_fast as fused_dual_window_attn_lse
from fused_conv import causal_dwconv_chunked
import fused_dual_attn, lse_dual_attn, fused_conv
kinds = {inspect.Parameter.POSITIONAL_OR_KEYWORD: "P", inspect.Parameter.KEYWORD_ONLY: "K",
         inspect.Parameter.POSITIONAL_ONLY: "O", inspect.Parameter.VAR_POSITIONAL: "*",
         inspect.Parameter.VAR_KEYWORD: "**"}
for mod, fn in json.loads(sys.argv[2]):
    f = getattr(sys.modules[mod], fn)
    ps = []
    for p in inspect.signature(f).parameters.values():
        d = "-" if p.default is inspect.Parameter.empty else repr(p.default)
        ps.append((p.name, kinds[p.kind], d))
    out[mod + "." + fn] = {"params": ps, "module": f.__module__,
                           "file": sys.modules[mod].__file__}
out["alias_is_fa3_fast"] = fused_dual_window_attn_lse is lse_dual_attn.lse_dual_window_attn_fa3_fast
print(json.dumps(out))
"""


def _probe():
    keys = [list(k) for k in REFERENCE_SIGNATURES]
    env = dict(os.environ)
    # only the drop-in directory: the modules must find the package themselves
    env.pop("PYTHONPATH", None)
    res = subprocess.run([sys.executable, "-c", _PROBE, DROPIN, json.dumps(keys)],
                         capture_output=True, text=True, cwd="/", env=env, timeout=300)
    assert res.returncode == 0, res.stderr
    return json.loads(res.stdout.strip().splitlines()[-1])


@pytest.fixture(scope="module")
def probed():
    return _probe()


@pytest.mark.parametrize("key", list(REFERENCE_SIGNATURES), ids=lambda k: ".".join(k))
def test_bare_name_signature_matches_reference(probed, key):
    got = probed[".".join(key)]
    ref = REFERENCE_SIGNATURES[key]
    params = [tuple(p) for p in got["params"]]
    assert params[:len(ref)] == ref, (params, ref)
    for name, kind, default in params[len(ref):]:
        assert kind == "K" and default != "-", f"extension {name} must be keyword-only with a default"
    # resolved from the drop-in directory and implemented by the HIP package
    assert os.path.dirname(got["file"]) == DROPIN
    assert got["module"].startswith("ttcd_amd.")


def test_patches_alias_import(probed):
    """patches.py:229 binds lse_dual_window_attn_fa3_fast under the fused name."""
    assert probed["alias_is_fa3_fast"]


def test_reference_error_conventions():
    """The reference's assertion errors (fused_dual_attn.py:256,
    lse_dual_attn.py:20) are raised before any device work, so they hold on
    CPU tensors too."""
    import torch

    sys.path.insert(0, DROPIN)
    try:
        from fused_dual_attn import fused_dual_window_attn
        from lse_dual_attn import lse_dual_window_attn
    finally:
        sys.path.remove(DROPIN)
    q = torch.zeros(1, 256, 2, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 256, 1, 64, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        fused_dual_window_attn(q, k, k, 128, 129)
    with pytest.raises(AssertionError):
        lse_dual_window_attn(q, k, k, 128, 128)


@pytest.mark.gpu
def test_bare_name_calls_match_package_calls_bitwise(gpu):
    """The three imports of patches.py resolve to the HIP kernels: each call
    through them is bit-identical to the same ttcd_amd call."""
    import torch

    from conftest import make_qkv
    from ttcd_amd import attn, conv

    sys.path.insert(0, DROPIN)
    try:
        from fused_conv import causal_dwconv_chunked
        from fused_dual_attn import fused_dual_window_attn
        from lse_dual_attn import lse_dual_window_attn_fa3_fast
    finally:
        sys.path.remove(DROPIN)
    q, k, v = make_qkv(batch=1, seqlen=1000, heads=4, kv_heads=2, head_dim=128, seed=3,
                       device=gpu)
    with torch.no_grad():
        ot, os_ = fused_dual_window_attn(q, k, v, 512, 256)
        rt, rs = attn.fused_dual_window_attn(q, k, v, 512, 256)
        assert torch.equal(ot, rt) and torch.equal(os_, rs)
        lt, ls = lse_dual_window_attn_fa3_fast(q, k, v, 512, 256)
        rlt, rls = attn.lse_dual_window_attn(q, k, v, 512, 256)
        assert torch.equal(lt, rlt) and torch.equal(ls, rls)
        g = torch.Generator().manual_seed(5)
        x = torch.randn(1, 3, 256, 384, generator=g).to(torch.bfloat16).to(gpu)
        c = torch.nn.Conv1d(384, 384, 5, groups=384, bias=False).to(gpu, torch.bfloat16)
        assert torch.equal(causal_dwconv_chunked(x, c), conv.causal_dwconv_chunked(x, c))
    torch.cuda.synchronize()
