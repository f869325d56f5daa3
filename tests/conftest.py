"""Shared pytest setup: the `gpu` marker, repo root on sys.path, seeded inputs."""
from __future__ import annotations

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")


def random_cases(default: int) -> int:
    """Case count of a seeded random sweep: `default`, times TTCD_RANDOM_SCALE when set
    (a one-off deeper check over the same seeds plus more)."""
    return max(1, int(default * float(os.environ.get("TTCD_RANDOM_SCALE", "1"))))


def make_qkv(*, batch, seqlen, heads, kv_heads, head_dim, dtype=torch.bfloat16, seed=0,
             qk_scale=1.0, device="cuda"):
    """Seeded N(0,1) q, k, v drawn on the CPU in the order q, k, v, then moved to `device`
    (the reference draws them with a cuda Generator; CPU draws keep the inputs identical on
    every machine). q and k are multiplied by qk_scale as in
    test/test_fused_dual_attn.py:34-75."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, seqlen, heads, head_dim, generator=g, dtype=torch.float32).to(dtype)
    k = torch.randn(batch, seqlen, kv_heads, head_dim, generator=g, dtype=torch.float32).to(dtype)
    v = torch.randn(batch, seqlen, kv_heads, head_dim, generator=g, dtype=torch.float32).to(dtype)
    if qk_scale != 1.0:
        q = (q.float() * qk_scale).to(dtype)
        k = (k.float() * qk_scale).to(dtype)
    return q.to(device), k.to(device), v.to(device)


@pytest.fixture(scope="session")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from ttcd_amd import _lib
    _lib.lib()  # fail loudly if the extension is missing on a GPU box
    return torch.device("cuda:0")
