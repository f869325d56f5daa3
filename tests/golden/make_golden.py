"""Writes tests/golden/golden_small.npz: small seeded inputs and the oracle's outputs.

Inputs are stored as raw bf16 bit patterns (int16). The vectors come from this
repository's CPU oracle (the reference ships no vectors for this path and its
kernels cannot run here); tests/test_oracle.py re-derives them to catch drift.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attn_ref, conv_ref  # noqa: E402


def main():
    g = torch.Generator().manual_seed(2026)
    B, T, H, HK, D, wt, ws = 1, 96, 4, 2, 32, 48, 20
    q = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, T, HK, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, T, HK, D, generator=g).to(torch.bfloat16)
    x = torch.randn(1, 2, 24, 16, generator=g).to(torch.bfloat16)
    w = torch.randn(16, 5, generator=g).to(torch.bfloat16)
    bits = lambda t: t.view(torch.int16).numpy()  # noqa: E731
    np.savez_compressed(
        os.path.join(HERE, "golden_small.npz"),
        q=bits(q), k=bits(k), v=bits(v), wt=np.int64(wt), ws=np.int64(ws),
        o_teacher=attn_ref.dense_reference(q, k, v, wt).numpy(),
        o_student=attn_ref.dense_reference(q, k, v, ws).numpy(),
        conv_x=bits(x), conv_w=bits(w), conv_y=conv_ref.dwconv_c(x, w).view(torch.int16).numpy(),
    )


if __name__ == "__main__":
    main()
