"""GPU chunked causal depthwise conv: bitwise equal to the fixed-order fp32 oracle
(profiling/fused_conv.py:39-48; REPORT.md:313 claims bitwise equality with cuDNN)."""
from __future__ import annotations

import pytest
import torch

from conftest import random_cases

from oracle import conv_ref

pytestmark = pytest.mark.gpu


def _run(x, w):
    from ttcd_amd import causal_dwconv_x
    return causal_dwconv_x(x.cuda(), w.cuda()).cpu()


def _bits_equal(a, b):
    return torch.equal(a.view(torch.int16) if a.dtype != torch.float32 else a.view(torch.int32),
                       b.view(torch.int16) if b.dtype != torch.float32 else b.view(torch.int32))


@pytest.mark.parametrize("shape,K,xdt,wdt", [
    ((1, 2, 256, 3072), 5, torch.bfloat16, torch.bfloat16),
    ((2, 3, 33, 24), 5, torch.bfloat16, torch.bfloat16),
    ((1, 1, 40, 20), 5, torch.bfloat16, torch.bfloat16),      # D % 8 != 0: scalar kernel
    ((1, 4, 17, 64), 1, torch.bfloat16, torch.bfloat16),
    ((1, 4, 17, 64), 3, torch.float16, torch.float16),
    ((1, 4, 70, 64), 7, torch.bfloat16, torch.float32),
    ((1, 4, 70, 64), 8, torch.float32, torch.float32),
    ((1, 2, 50, 32), 9, torch.bfloat16, torch.bfloat16),       # K > 8: scalar kernel
    ((1, 2, 3, 32), 5, torch.bfloat16, torch.bfloat16),        # C < K
])
@torch.inference_mode()
def test_bitwise_vs_oracle(gpu, shape, K, xdt, wdt):
    g = torch.Generator().manual_seed(sum(shape) + K)
    x = torch.randn(*shape, generator=g).to(xdt)
    w = torch.randn(shape[-1], K, generator=g).to(wdt)
    y = _run(x, w)
    assert _bits_equal(y, conv_ref.dwconv_c(x, w))


@torch.inference_mode()
def test_full_shape_bitwise(gpu):
    """The reference's conv benchmark shape x = (1, 16, 4096, 3072) bf16, K = 5
    (profiling/fused_conv.py:77)."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 16, 4096, 3072, generator=g).to(torch.bfloat16)
    w = torch.randn(3072, 5, generator=g).to(torch.bfloat16)
    assert _bits_equal(_run(x, w), conv_ref.dwconv_c(x, w))


@torch.inference_mode()
def test_module_api_and_identity_init(gpu):
    """causal_dwconv_chunked(x, conv) with the model's identity init (tap K-1 = 1,
    modeling_ipttcdv9.py:977-994) returns x exactly."""
    from ttcd_amd import causal_dwconv_chunked
    D, K = 96, 5
    conv = torch.nn.Conv1d(D, D, K, padding=0, groups=D, bias=False)
    with torch.no_grad():
        conv.weight.zero_()
        conv.weight[:, 0, K - 1] = 1.0
    conv = conv.cuda().to(torch.bfloat16)
    x = torch.randn(2, 3, 64, D).to(torch.bfloat16).cuda()
    assert torch.equal(causal_dwconv_chunked(x, conv), x)


def _random_conv_case(i):
    import random
    r = random.Random(500 + i)
    b, nch = r.randint(1, 3), r.randint(1, 4)
    C = r.choice([1, 2, r.randint(1, 40), r.randint(16, 300)])
    D = r.choice([8, 16, 24, 64, 136, 3072, r.randint(1, 200)])
    K = r.choice([1, 2, 3, 4, 5, 5, 6, 7, 8, r.randint(9, 64)])
    xdt = r.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    wdt = r.choice([xdt, torch.float32, torch.bfloat16])
    return (b, nch, C, D), K, xdt, wdt


@pytest.mark.parametrize("i", range(random_cases(60)))
@torch.inference_mode()
def test_random_shapes_bitwise_vs_oracle(gpu, i):
    """Seeded random shapes (vector and scalar kernels, K up to 64, every dtype pair)
    bitwise against the fixed-order oracle."""
    shape, K, xdt, wdt = _random_conv_case(i)
    print(f"case {i}: shape {shape} K {K} x {xdt} w {wdt}", flush=True)
    g = torch.Generator().manual_seed(900 + i)
    x = torch.randn(*shape, generator=g).to(xdt)
    w = torch.randn(shape[-1], K, generator=g).to(wdt)
    assert _bits_equal(_run(x, w), conv_ref.dwconv_c(x, w)), f"case {i}"
