"""CPU oracle for the chunked causal depthwise conv (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker.

  dwconv_c          - ctypes binding of oracle/conv_oracle.c (fixed-order fmaf
                      accumulation, RNE rounding; any of bf16/f16/f32 for x and w).
                      Restates profiling/fused_conv.py:39-48 and :56-58.
  dwconv_numpy      - numpy float32 restatement of the same loop (16-bit weights:
                      every product is exact in fp32, so mul+add == fmaf).
  conv1d_reference  - IPTTCDMLP._apply_ttt_conv's formulation
                      (custom_models/ipttcd/modeling_ipttcdv9.py:203-211:
                      rearrange, left pad K-1, depthwise conv1d, rearrange back)
                      evaluated in float64 with torch.nn.functional.conv1d.

Pins (tests/test_oracle.py): dwconv_c == dwconv_numpy bit for bit; both ==
conv1d_reference rounded once (exact products, sums checked against the fp64
conv within one rounding); identity weight (tap K-1 = 1) reproduces x; the
C encoders (bf16 / f16 RNE) agree with torch's casts on every tested value.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np
import torch
import torch.nn.functional as F

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "libttcd_oracle.so")
_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
_lock = threading.Lock()
_lib = None


def build() -> str:
    """make -C oracle (gcc); idempotent."""
    subprocess.run(["make", "-s", "-C", _DIR], check=True, capture_output=True)
    return LIB_PATH


def _load():
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                build()
            lib = ctypes.CDLL(LIB_PATH)
            lib.ttcd_oracle_dwconv.restype = None
            lib.ttcd_oracle_dwconv.argtypes = [
                ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int]
            lib.ttcd_oracle_round.restype = None
            lib.ttcd_oracle_round.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                              ctypes.c_int64]
            _lib = lib
    return _lib


def dwconv_c(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x (..., C, D) CPU tensor, w (D, K): fixed-order fp32 conv, rounded to x.dtype."""
    lib = _load()
    x = x.detach().cpu().contiguous()
    w = w.detach().cpu().contiguous()
    C, D = x.shape[-2], x.shape[-1]
    K = w.shape[1]
    N = x.numel() // (C * D) if C * D else 0
    y = torch.empty_like(x)
    lib.ttcd_oracle_dwconv(x.data_ptr(), _CODES[x.dtype], w.data_ptr(), _CODES[w.dtype],
                           y.data_ptr(), N, C, D, K)
    return y


def round_c(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """fp32 -> dtype through the oracle's own RNE encoders."""
    lib = _load()
    src = x.detach().cpu().float().contiguous()
    out = torch.empty(src.shape, dtype=dtype)
    lib.ttcd_oracle_round(src.data_ptr(), out.data_ptr(), _CODES[dtype], src.numel())
    return out


def dwconv_numpy(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Same loop in numpy float32 (valid bit-exactly when w is 16-bit)."""
    assert w.dtype in (torch.bfloat16, torch.float16), "fp32 weights need the fmaf oracle"
    xs = x.detach().cpu().float().numpy()
    ws = w.detach().cpu().float().numpy()  # (D, K)
    C = xs.shape[-2]
    K = ws.shape[1]
    acc = np.zeros_like(xs, dtype=np.float32)
    for j in range(K):
        shift = K - 1 - j
        src = np.zeros_like(xs)
        if shift < C:
            src[..., shift:, :] = xs[..., :C - shift, :]
        acc = (acc + src * ws[:, j].astype(np.float32)).astype(np.float32)
    return torch.from_numpy(acc).to(x.dtype)


def conv1d_reference(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """The model's rearrange -> pad -> depthwise conv1d -> rearrange, in float64."""
    D, K = w.shape
    lead = x.shape[:-2]
    C = x.shape[-2]
    xf = x.detach().cpu().double().reshape(-1, C, D).transpose(1, 2)  # (n, D, C)
    xf = F.pad(xf, (K - 1, 0))
    y = F.conv1d(xf, w.detach().cpu().double().view(D, 1, K), groups=D)
    return y.transpose(1, 2).reshape(*lead, C, D)
