"""Writes tests/golden/golden_small.npz (small seeded inputs and the oracle's
outputs, D=32) and tests/golden/golden_attn.npz (the kernels' head sizes, D=64
and D=128, GQA group 2, both windows truncating: the oracle's fp32 outputs and
LSEs for both windows).

Inputs are stored as raw bf16 bit patterns (int16). The vectors come from this
repository's CPU oracle (the reference ships no vectors for this path and its
kernels cannot run here); tests/test_oracle.py re-derives them to catch drift,
and tests/test_golden_gpu.py holds the GPU kernels to them.

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


def attn_cases():
    """(name, B, T, H, HK, D, wt, ws, seed) of golden_attn.npz."""
    return [("d64", 1, 128, 2, 1, 64, 96, 40, 7), ("d128", 1, 112, 2, 1, 128, 72, 33, 8)]


def main_attn():
    bits = lambda t: t.view(torch.int16).numpy()  # noqa: E731
    arrays = {}
    for name, B, T, H, HK, D, wt, ws, seed in attn_cases():
        g = torch.Generator().manual_seed(seed)
        q = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16)
        k = torch.randn(B, T, HK, D, generator=g).to(torch.bfloat16)
        v = torch.randn(B, T, HK, D, generator=g).to(torch.bfloat16)
        ot, lt = attn_ref.dense_reference(q, k, v, wt, return_lse=True)
        os_, ls = attn_ref.dense_reference(q, k, v, ws, return_lse=True)
        arrays.update({f"{name}_q": bits(q), f"{name}_k": bits(k), f"{name}_v": bits(v),
                       f"{name}_windows": np.array([wt, ws], dtype=np.int64),
                       f"{name}_o_teacher": ot.numpy(), f"{name}_o_student": os_.numpy(),
                       f"{name}_lse_teacher": lt.numpy(), f"{name}_lse_student": ls.numpy()})
    np.savez_compressed(os.path.join(HERE, "golden_attn.npz"), **arrays)


if __name__ == "__main__":
    main()
    main_attn()
