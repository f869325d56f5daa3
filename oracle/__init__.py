"""CPU oracle for the dual-window attention / LSE merge / chunked conv path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this package, and only as the
checker; the product path (ttcd_amd) never routes through it.

Modules
  attn_ref  - fp32 masked-softmax attention (dense and banded), LSE, LSE
              merge, a numerics emulator of the reference Triton kernel, the
              bf16 ULP report, band pair / FLOP counts.
  conv_ref  - fixed-order fp32 depthwise causal conv: numpy restatement,
              ctypes binding of the C restatement (conv_oracle.c, built by
              oracle/Makefile into oracle/libttcd_oracle.so), and the
              reference model's Conv1d formulation.

Parity pins (what each function is checked against) are listed in each
module's docstring; none of them is "parity unpinned".

No reference C/C++ sources exist for this path (the reference is Python +
Triton), so there is no oracle/_ref build.
"""
