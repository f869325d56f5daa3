#!/usr/bin/env python3
"""Benchmark of the MI355X dual-window attention hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config qwen3|smollm2]

A "step" is one call of fused_dual_window_attn on the Qwen3-0.6B 64K layer
shape (B=1, T=65536, Hq=16, Hkv=8, D=128, w_T=8192, w_S=4096), producing the
teacher and student outputs plus both per-row LSEs, with q/k/v (bf16 N(0,1),
seed 0) already resident in HBM. `value` is TFLOP/s over the teacher band's
algorithmic FLOPs F = 4*B*Hq*D*P(T, w_T) (the student band is reused, not
counted), timed with HIP events on the launch stream over exactly K steps.

Prints progress on stderr and ONE JSON line on stdout. Beside the headline
it reports: the "two separate windowed calls" comparator (the single-band
kernel at w_T then w_S), one teacher-only call, the LSE-combination variant,
the chunked causal conv at the reference's benchmark shape (GB/s vs 8 TB/s),
the attention prologue (q/k RMSNorm + rotary) and epilogue (o_proj + dual
residual RMSNorm) on the same layer, the reference's other 64K window recipes
(2048/1024 and 16384/8192), the fused outputs against the single-band kernel
on every row (bit-equal fraction), full causal attention against torch's SDPA
flash backend on the same tensors, the batch / narrow-gap sweep (fused vs
LSE variant), the ipttcdv9 prefill end to end (28 layers, T=32768; fused,
patched and stock paths; and T=65536, the length of the reference's published
end-to-end numbers, in one call and in four 16K chunks over the K/V cache),
numerics at the CPU-runnable config and on sampled query blocks of the
headline shape, and the CPU baseline: the fp32 masked
softmax of the reference's CPU path (oracle restatement), query-chunked over
the band, on a bounded sample of rows, on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
import types

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "dual-window attn prefill TFLOP/s + % bf16 MFMA peak, Qwen3-0.6B 64K"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E

CONFIGS = {
    # rope_theta / qk_norm / hidden / norm_eps:
    # configs/ipttcd/ipttcdv9_qwen3_0.6B_ct_64k_v2_swa8k.json:3,11,14,18 and
    # configs/ipttcd/ipttcdv9_smollm2_360M_ct_64k_v2_swa8k.json:3,11,14,18
    "qwen3": dict(name="Qwen3-0.6B layer, 64K prefill", B=1, T=65536, Hq=16, Hkv=8, D=128,
                  wt=8192, ws=4096, rope_theta=1e6, qk_norm=True, hidden=1024, norm_eps=1e-6),
    "smollm2": dict(name="SmolLM2-360M layer, 64K prefill", B=1, T=65536, Hq=15, Hkv=5, D=64,
                    wt=8192, ws=4096, rope_theta=1e5, qk_norm=False, hidden=960, norm_eps=1e-5),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_gpu(fn, steps: int, warmup: int, min_warm_s: float = 0.2) -> float:
    """Mean ms per call over `steps` calls, HIP events on the current (launch) stream.
    Warm-up is `warmup` calls and at least `min_warm_s` of back-to-back work: a
    short kernel timed right after the GPU idled runs up to 18 % slow (measured
    for the 1 ms B=1, T=16384 sweep point) while the clocks ramp."""
    import torch
    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < min_warm_s:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def cpu_baseline(q, k, v, cfg, target_s: float) -> dict:
    """fp32 masked-softmax attention of the reference's CPU path
    (test/test_fused_dual_attn.py:88-110, one call per window: teacher then
    student), query-chunked over the band, on a run of full-window rows."""
    import torch
    from oracle import attn_ref

    # every core this process may run on (the box's CPU share)
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    B, T, H, D, wt, ws = cfg["B"], cfg["T"], cfg["Hq"], cfg["D"], cfg["wt"], cfg["ws"]
    r0 = T // 2
    span = 8192
    qc = q[:, r0:r0 + span].cpu()
    kc = k[:, r0 - wt + 1:r0 + span].cpu()
    vc = v[:, r0 - wt + 1:r0 + span].cpu()
    off = wt - 1  # row r0 + i of the full tensors is row off + i of the key slice

    def run(n):
        rows = torch.arange(off, off + n)
        qpad = torch.zeros(B, off + n, H, D, dtype=qc.dtype)
        qpad[:, off:] = qc[:, :n]
        for W in (wt, ws):
            attn_ref.band_reference(qpad, kc[:, :off + n], vc[:, :off + n], 0, W, rows=rows)

    # Size the sample from a warm 128-row probe (the first call also pays for
    # thread start-up and allocation), so the four timed-or-warm-up runs take
    # about target_s together.
    run(128)
    t0 = time.perf_counter()
    run(128)
    t128 = time.perf_counter() - t0
    n = int(min(span, max(64, round(128 * (target_s / 4) / max(t128, 1e-3) / 64) * 64)))
    run(n)  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run(n)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    flops = 4 * B * H * D * wt * n  # teacher-band FLOPs of n full-window rows (same F)
    cpu_model = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                cpu_model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": flops / t / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{n} consecutive query rows x {H} heads at t={r0}.. (full {wt}-key windows), "
                   f"fp32 masked softmax per window (teacher {wt} then student {ws}), "
                   f"query-chunked over the band (dense form needs {B*H*T*T*4/1e9:.0f} GB); "
                   f"median of 3 runs after 1 warm-up, {t:.2f} s/run"),
        "tokens_per_s": B * n / t,
        "threads_source": "len(os.sched_getaffinity(0))",
        "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"),
        "os_cpu_count": os.cpu_count(),
        "cpu_model": cpu_model or platform.processor(),
    }


def numerics_report(D: int = 64) -> dict:
    """Config 1 (B=1, T=2048, Hq=4, Hkv=2, D=64, 512/256; D=128 for the head
    size whose lazy rescale follows the tile-sum rule): GPU vs fp32 oracle and the
    fraction of bf16 outputs bit-identical to a CPU emulation of the reference kernel,
    for the default lazy rescale and for exact_max=True (the reference's exact running
    max)."""
    import torch
    from oracle import attn_ref
    from ttcd_amd import fused_dual_window_attn

    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 2048, 4, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 2048, 2, D, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 2048, 2, D, generator=g).to(torch.bfloat16)
    with torch.inference_mode():
        ot, os_ = fused_dual_window_attn(q.cuda(), k.cuda(), v.cuda(), 512, 256)
        xt, xs = fused_dual_window_attn(q.cuda(), k.cuda(), v.cuda(), 512, 256, exact_max=True)
    et, es = attn_ref.emulate_reference_kernel(q, k, v, 512, 256)
    out = {}
    for name, o, x, e, W in (("teacher", ot, xt, et, 512), ("student", os_, xs, es, 256)):
        o, x = o.cpu(), x.cpu()
        ref = attn_ref.dense_reference(q, k, v, W)
        mx, mean = attn_ref.error_stats(o, ref)
        rep = attn_ref.ulp_report(o, e)
        rep_x = attn_ref.ulp_report(x, e)
        out[name] = {"max_abs_err_vs_fp32": mx, "mean_abs_err_vs_fp32": mean,
                     "bit_identical_to_ref_kernel_emulation_pct": rep["bit_equal_pct"],
                     "le1ulp_pct": rep["le1ulp_pct"], "max_ulp": rep["max_ulp"],
                     "exact_max": {"max_abs_err_vs_fp32": attn_ref.error_stats(x, ref)[0],
                                   "bit_identical_to_ref_kernel_emulation_pct":
                                       rep_x["bit_equal_pct"],
                                   "le1ulp_pct": rep_x["le1ulp_pct"]}}
    return out


RECIPES_64K = [
    # the reference's other published windows at T = 65536, Qwen3 heads, with its
    # own H100 timings (profiling/fused_dual_attn.py:295, profiling/REPORT.md:252-253)
    dict(wt=2048, ws=1024, ref_h100_fused_ms=3.6, ref_h100_two_calls_ms=5.7),
    dict(wt=16384, ws=8192, ref_h100_fused_ms=22.5, ref_h100_two_calls_ms=37.7),
]


def recipes_measure(q, k, v, steps: int = 10, warmup: int = 3) -> list:
    """The other 64K window recipes on the headline tensors: the fused call (with
    both LSEs), the two separate windowed calls and the LSE variant; TFLOP/s over
    the teacher band as the headline."""
    from ttcd_amd import fused_dual_window_attn, lse_dual_window_attn, window_attn, work as W

    B, T, H, D = q.shape
    out = []
    for r in RECIPES_64K:
        wt, ws = r["wt"], r["ws"]
        F, F_s = W.attn_flops(B, H, D, T, wt), W.attn_flops(B, H, D, T, ws)
        ms = time_gpu(lambda: fused_dual_window_attn(q, k, v, wt, ws, return_lse=True),
                      steps, warmup)
        ms_two = time_gpu(lambda: (window_attn(q, k, v, wt), window_attn(q, k, v, ws)),
                          steps, 2)
        ms_lse = time_gpu(lambda: lse_dual_window_attn(q, k, v, wt, ws), steps, 2)
        tf = F / (ms * 1e-3) / 1e12
        log(f"recipe ({wt}, {ws}): fused {ms:.3f} ms {tf:.0f} TF/s "
            f"({100 * tf / PEAK_BF16_TFLOPS:.1f}%), two calls {ms_two:.3f} ms, "
            f"LSE variant {ms_lse:.3f} ms")
        out.append({"window_teacher": wt, "window_student": ws, "T": T, "flops": F, "ms": ms,
                    "tflops": tf, "frac_of_bf16_peak": tf / PEAK_BF16_TFLOPS,
                    "two_separate_calls_ms": ms_two, "fused_speedup_vs_two_calls": ms_two / ms,
                    "ideal_speedup_vs_two_calls": (F + F_s) / F, "lse_variant_ms": ms_lse,
                    "fused_speedup_vs_lse": ms_lse / ms,
                    "reference_h100_ms": {"fused": r["ref_h100_fused_ms"],
                                          "two_calls": r["ref_h100_two_calls_ms"],
                                          "source": "profiling/REPORT.md:252-253"}})
    return out


def vendor_sdpa_measure(q, k, v, steps: int = 5, warmup: int = 2) -> dict:
    """The vendor attention on this box as a yardstick: torch's
    scaled_dot_product_attention with its flash backend (AOTriton on ROCm) on
    full causal attention over the headline tensors, against this library's
    single-band kernel on the same problem (window = T). PyTorch has no sliding
    window, so full causal is the problem both can run; the FLOPs are equal.
    SDPA gets contiguous (B, H, T, D) copies made outside the timed region."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from ttcd_amd import window_attn, work as W

    B, T, H, D = q.shape
    HK = k.shape[2]
    F = W.attn_flops(B, H, D, T, None)
    ms_own = time_gpu(lambda: window_attn(q, k, v, None), steps, warmup)
    o_own = window_attn(q, k, v, None)
    qh, kh, vh = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    sdpa = lambda: torch.nn.functional.scaled_dot_product_attention(  # noqa: E731
        qh, kh, vh, is_causal=True, enable_gqa=HK != H)
    out = {"problem": f"full causal, B={B} T={T} Hq={H} Hkv={HK} D={D}, bf16", "flops": F,
           "own_ms": ms_own, "own_tflops": F / (ms_own * 1e-3) / 1e12,
           "torch_version": torch.__version__}
    try:
        with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
            o_v = sdpa()
            ms_v = time_gpu(sdpa, steps, warmup)
        out.update({"sdpa_backend": "flash", "sdpa_ms": ms_v,
                    "sdpa_tflops": F / (ms_v * 1e-3) / 1e12, "own_speedup": ms_v / ms_own,
                    "max_abs_diff": (o_v.transpose(1, 2).float() - o_own.float()).abs().max().item()})
        del o_v
    except RuntimeError as e:  # no flash kernel for this build / shape
        out.update({"sdpa_backend": None, "sdpa_error": str(e)[:200]})
    log(f"vendor SDPA yardstick: {out}")
    return out


def second_kernel_agreement(q, k, v, wt, ws) -> dict:
    """The fused outputs on every row against the single-band kernel at each window
    (the reference's fused-vs-flash-attention comparison, profiling/REPORT.md:248:
    99.7-99.9 % bit-equal there), in both rescale modes."""
    import torch
    from ttcd_amd import fused_dual_window_attn, window_attn

    def pct(a, b):
        return 100.0 * (a.view(torch.int16) == b.view(torch.int16)).float().mean().item()

    out = {}
    for exact in (False, True):
        ot, os_ = fused_dual_window_attn(q, k, v, wt, ws, exact_max=exact)
        rep = {}
        for name, o, W in (("teacher", ot, wt), ("student", os_, ws)):
            second = window_attn(q, k, v, W, exact_max=exact)
            d = (o.float() - second.float()).abs()
            rep[name] = {"bit_equal_pct": pct(o, second), "max_abs": d.max().item(),
                         "mean_abs": d.mean().item()}
            del second, d
        out["exact_max" if exact else "lazy"] = rep
        del ot, os_
    out["note"] = ("all rows; second kernel = ttcd_band_attn_fwd at w_T, then at w_S, same "
                   "rescale mode; the reference test's bounds are max <= 2e-3, mean <= 2e-6 "
                   "(test/test_fused_dual_attn.py:385-402)")
    return out


HEADLINE_SAMPLE_BLOCKS = (0, 4032, 4096, 8128, 8192, 20032, 40000, 65472)
HEADLINE_SAMPLE_HEADS = (0, 5, 10, 15)


def numerics_headline(q, k, v, wt, ws) -> dict:
    """Headline-shape numerics: fraction of bf16 outputs bit-identical to the CPU
    emulation of the reference kernel (oracle/attn_ref.py:emulate_reference_kernel),
    lazy and exact_max, on sampled 64-row query blocks (around 0, w_S, w_T, the
    middle and the tail) x sampled heads; the emulation of all rows would take
    hours on the CPU."""
    import torch
    from oracle import attn_ref
    from ttcd_amd import fused_dual_window_attn

    blocks = [b - b % 64 for b in HEADLINE_SAMPLE_BLOCKS]
    heads = list(HEADLINE_SAMPLE_HEADS)
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    t0 = time.perf_counter()
    et, es = attn_ref.emulate_reference_kernel(qc, kc, vc, wt, ws, row_blocks=blocks,
                                               heads=heads)
    t_emul = time.perf_counter() - t0
    rows = torch.cat([torch.arange(b, min(b + 64, q.shape[1])) for b in blocks])
    hs = torch.tensor(heads)
    out = {"sample": f"query blocks starting at {blocks} x heads {heads} "
                     f"({len(blocks) * len(heads)} blocks of 64 rows x 128 values)",
           "emulation_s": t_emul}
    for exact in (False, True):
        ot, os_ = fused_dual_window_attn(q, k, v, wt, ws, exact_max=exact)
        rep = {}
        for name, o, e in (("teacher", ot, et), ("student", os_, es)):
            a = o.cpu()[:, rows][:, :, hs]
            r = attn_ref.ulp_report(a, e[:, rows][:, :, hs])
            rep[name] = {"bit_identical_to_ref_kernel_emulation_pct": r["bit_equal_pct"],
                         "le1ulp_pct": r["le1ulp_pct"], "max_ulp": r["max_ulp"]}
        out["exact_max" if exact else "lazy"] = rep
    return out


def profile_one(args) -> int:
    """One workload, `--steps` timed launches after `--warmup`, for rocprofv3 runs.
    'copy' is a plain device-to-device copy of 1 GiB (the known-size kernel used to
    calibrate the FETCH_SIZE / WRITE_SIZE counters)."""
    import torch
    from ttcd_amd import causal_dwconv_x, fused_dual_window_attn, lse_dual_window_attn, window_attn
    from ttcd_amd import work as W

    dev = torch.device("cuda:0")
    cfg = CONFIGS[args.config]
    B, T, H, HK, D, wt, ws = (cfg[k] for k in ("B", "T", "Hq", "Hkv", "D", "wt", "ws"))
    gen = torch.Generator(device=dev).manual_seed(0)
    if args.only == "prologue":
        q = torch.randn(B, T, H, D, device=dev, dtype=torch.bfloat16, generator=gen)
        k = torch.randn(B, T, HK, D, device=dev, dtype=torch.bfloat16, generator=gen)
        from ttcd_amd import prologue
        w = torch.ones(D, device=dev, dtype=torch.bfloat16)
        cos, sin = prologue.rope_tables(prologue.rope_inv_freq(D, cfg["rope_theta"], dev), T)
        norm = cfg["qk_norm"]
        fn = lambda: prologue.qk_norm_rope(q, k, w if norm else None, w if norm else None,  # noqa: E731
                                           1e-5, cos, sin)
        work, unit = W.prologue_bytes(B, T, H, HK, D), "GB/s"
    elif args.only == "epilogue":
        from ttcd_amd import epilogue
        Hd = cfg["hidden"]
        a_t, a_s, r = (torch.randn(B, T, Hd, device=dev, dtype=torch.bfloat16, generator=gen)
                       for _ in range(3))
        w = torch.ones(Hd, device=dev, dtype=torch.bfloat16)
        fn = lambda: epilogue.dual_residual_rmsnorm(a_t, a_s, r, w, cfg["norm_eps"])  # noqa: E731
        work, unit = W.epilogue_bytes(B * T, Hd), "GB/s"
    elif args.only == "copy":
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        fn, work, unit = (lambda: dst.copy_(src)), float(1 << 31), "GB/s"
    elif args.only == "conv":
        x = torch.randn(1, 16, 4096, 3072, device=dev, dtype=torch.bfloat16, generator=gen)
        w = torch.randn(3072, 5, device=dev, dtype=torch.bfloat16, generator=gen)
        fn, work, unit = (lambda: causal_dwconv_x(x, w)), W.conv_bytes(16, 4096, 3072, 5), "GB/s"
    else:
        q = torch.randn(B, T, H, D, device=dev, dtype=torch.bfloat16, generator=gen)
        k = torch.randn(B, T, HK, D, device=dev, dtype=torch.bfloat16, generator=gen)
        v = torch.randn(B, T, HK, D, device=dev, dtype=torch.bfloat16, generator=gen)
        work, unit = W.attn_flops(B, H, D, T, wt), "TFLOP/s"
        if args.only in ("causal", "sdpa"):
            # full causal: this library's single-band kernel, or torch's SDPA
            # flash backend on contiguous (B, H, T, D) copies
            work = W.attn_flops(B, H, D, T, None)
            if args.only == "causal":
                fn = lambda: window_attn(q, k, v, None)  # noqa: E731
            else:
                from torch.nn.attention import SDPBackend, sdpa_kernel
                qh, kh, vh = (t.transpose(1, 2).contiguous() for t in (q, k, v))

                def fn():
                    with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
                        return torch.nn.functional.scaled_dot_product_attention(
                            qh, kh, vh, is_causal=True, enable_gqa=HK != H)
        elif args.only == "fused":
            fn = lambda: fused_dual_window_attn(q, k, v, wt, ws, return_lse=True)  # noqa: E731
        elif args.only == "band":
            fn = lambda: window_attn(q, k, v, wt)  # noqa: E731
        else:
            fn = lambda: lse_dual_window_attn(q, k, v, wt, ws)  # noqa: E731
    with torch.inference_mode():
        ms = time_gpu(fn, args.steps, args.warmup)
    rate = work / (ms * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9)
    print(json.dumps({"only": args.only, "config": args.config, "ms": ms, "rate": rate,
                      "unit": unit, "steps": args.steps}), flush=True)
    return 0


def prologue_measure(q, k, cfg) -> dict:
    """The attention prologue (q/k RMSNorm + rotary, one pass) on the bench's own
    q and k: HBM-bound, so GB/s against the 8 TB/s peak."""
    import torch
    from ttcd_amd import prologue, work as W

    B, T, H, HK, D = q.shape[0], q.shape[1], q.shape[2], k.shape[2], q.shape[3]
    dev = q.device
    wq = (1.0 + 0.1 * torch.randn(D, device=dev, generator=torch.Generator(device=dev)
                                  .manual_seed(1))).to(torch.bfloat16)
    cos, sin = prologue.rope_tables(prologue.rope_inv_freq(D, cfg["rope_theta"], dev), T)
    norm = cfg["qk_norm"]
    fn = lambda: prologue.qk_norm_rope(q, k, wq if norm else None, wq if norm else None,  # noqa: E731
                                       1e-5, cos, sin)
    ms_p = time_gpu(fn, 20, 3)
    nbytes = W.prologue_bytes(B, T, H, HK, D)
    gbps = nbytes / (ms_p * 1e-3) / 1e9
    qk_bytes = B * T * (H + HK) * D * 2
    table_bytes = 2 * T * (D // 2) * 2
    # the reference's launches: q_norm, k_norm (each a read and a write), then
    # rotary on q and on k (a read, a write and the table rows each)
    ref_bytes = (2 * qk_bytes if norm else 0) + 2 * qk_bytes + 2 * table_bytes
    return {"shape": {"B": B, "T": T, "Hq": H, "Hkv": HK, "D": D}, "qk_norm": norm,
            "rope_theta": cfg["rope_theta"], "ms": ms_p, "GB_per_s": gbps,
            "frac_of_hbm_peak": gbps / PEAK_HBM_GBPS, "algorithmic_bytes": nbytes,
            "reference_launches_bytes": ref_bytes}


SWEEP = [
    # the batch and narrow-gap sweep at the Qwen3-0.6B head shape (Hq=16, Hkv=8, D=128)
    dict(B=1, T=16384, wt=8192, ws=4096), dict(B=2, T=16384, wt=8192, ws=4096),
    dict(B=4, T=16384, wt=8192, ws=4096), dict(B=8, T=16384, wt=8192, ws=4096),
    dict(B=1, T=32768, wt=8192, ws=7168), dict(B=1, T=32768, wt=8192, ws=8064),
]


def sweep_measure(steps: int = 10, warmup: int = 2) -> list:
    """Fused one-pass kernel (with both LSEs, as the headline) against the
    LSE-combination variant at each sweep point; TFLOP/s over the teacher
    band F = 4*B*Hq*D*P(T, w_T) for both."""
    import torch
    from ttcd_amd import fused_dual_window_attn, lse_dual_window_attn, work as W

    dev = torch.device("cuda:0")
    H, HK, D = 16, 8, 128
    out = []
    for pt in SWEEP:
        B, T, wt, ws = pt["B"], pt["T"], pt["wt"], pt["ws"]
        gen = torch.Generator(device=dev).manual_seed(0)
        q = torch.randn(B, T, H, D, device=dev, dtype=torch.bfloat16, generator=gen)
        k = torch.randn(B, T, HK, D, device=dev, dtype=torch.bfloat16, generator=gen)
        v = torch.randn(B, T, HK, D, device=dev, dtype=torch.bfloat16, generator=gen)
        F = W.attn_flops(B, H, D, T, wt)
        ms_f = time_gpu(lambda: fused_dual_window_attn(q, k, v, wt, ws, return_lse=True),
                        steps, warmup)
        ms_l = time_gpu(lambda: lse_dual_window_attn(q, k, v, wt, ws), steps, warmup)
        tf, tl = F / (ms_f * 1e-3) / 1e12, F / (ms_l * 1e-3) / 1e12
        out.append({**pt, "Hq": H, "Hkv": HK, "D": D, "flops": F, "fused_ms": ms_f,
                    "fused_tflops": tf, "fused_frac": tf / PEAK_BF16_TFLOPS, "lse_ms": ms_l,
                    "lse_tflops": tl, "fused_speedup_vs_lse": ms_l / ms_f})
        log(f"sweep B={B} T={T} ({wt},{ws}): fused {ms_f:.3f} ms {tf:.0f} TF/s, "
            f"LSE {ms_l:.3f} ms {tl:.0f} TF/s")
        del q, k, v
    return out


E2E_T = 32768  # the e2e prefill length (config 5)


def e2e_measure(steps: int = 5, warmup: int = 2, T: int = E2E_T,
                paths=("fused", "patched", "stock")) -> dict:
    """Prefill of the ipttcdv9 model at the Qwen3-0.6B shape (28 layers, TTT
    layers 0/7/14/21, w_T 8192, w_S 4096, conv K=5 on 3072 channels),
    random-init weights (the reference's init, seed 0), uniform token ids
    (seed 1234), B=1, logits of the last token. Paths of the TTT layers:
    "stock" = the reference's unpatched fast path (two windowed calls, torch's
    conv); "patched" = its `--patch fused_conv` (one-pass dual-window kernel +
    conv kernel); "fused" = patched + the fused epilogue and feature pass."""
    import torch
    from ttcd_amd import ipttcdv9

    dev = torch.device("cuda:0")
    cfg = ipttcdv9.QWEN3_06B_SWA8K
    weights = ipttcdv9.init_weights(cfg, dev, seed=0)
    g = torch.Generator(device=dev).manual_seed(1234)
    ids = torch.randint(0, cfg["vocab_size"], (1, T), device=dev, generator=g)
    flops = ipttcdv9.prefill_flops(cfg, 1, T)
    total = sum(flops.values())
    out = {"model": "ipttcdv9, Qwen3-0.6B shape (configs/ipttcd/ipttcdv9_qwen3_0.6B_ct_64k_v2_swa8k.json)",
           "B": 1, "T": T, "logits_to_keep": 1, "flops": flops}
    for path in paths:
        model = ipttcdv9.IPTTCDv9Prefill(cfg, weights, path=path)
        ms = time_gpu(lambda: model.forward(ids), steps, warmup)
        out[path] = {"ms": ms, "tokens_per_s": T / (ms * 1e-3),
                     "tflops": total / (ms * 1e-3) / 1e12}
        log(f"e2e prefill T={T} {path}: {ms:.2f} ms, {T / (ms * 1e-3):.0f} tok/s")
        del model
    if "stock" in out:
        out["fused_speedup_vs_stock"] = out["stock"]["ms"] / out["fused"]["ms"]
    if "patched" in out:
        out["fused_speedup_vs_patched"] = out["patched"]["ms"] / out["fused"]["ms"]
    out["peak_mem_gb"] = torch.cuda.max_memory_allocated(dev) / 1e9
    return out


def e2e_chunked_measure(T: int = 65536, chunk: int = 16384, steps: int = 3,
                        warmup: int = 1) -> dict:
    """The same prefill (fused path, same weights and token ids as
    e2e_measure) in chunks over the K/V cache: T tokens as T / chunk calls of
    IPTTCDv9Prefill.forward sharing one IPTTCDv9Cache, so every attention
    call after the first runs Tq = chunk queries against the cached window.
    Timed over the whole prompt; logits of the last token."""
    import torch
    from ttcd_amd import ipttcdv9

    dev = torch.device("cuda:0")
    cfg = ipttcdv9.QWEN3_06B_SWA8K
    weights = ipttcdv9.init_weights(cfg, dev, seed=0)
    g = torch.Generator(device=dev).manual_seed(1234)
    ids = torch.randint(0, cfg["vocab_size"], (1, T), device=dev, generator=g)
    model = ipttcdv9.IPTTCDv9Prefill(cfg, weights, path="fused")

    def run():
        cache = ipttcdv9.IPTTCDv9Cache()
        for c0 in range(0, T, chunk):
            logits = model.forward(ids[:, c0:c0 + chunk], logits_to_keep=1, cache=cache)
        return logits

    with torch.inference_mode():
        ms = time_gpu(run, steps, warmup)
    log(f"e2e prefill T={T} in chunks of {chunk} over the cache: {ms:.2f} ms")
    return {"T": T, "chunk": chunk, "calls": -(-T // chunk), "path": "fused", "ms": ms,
            "tokens_per_s": T / (ms * 1e-3)}


def epilogue_measure(o_t, o_s, cfg) -> dict:
    """The attention epilogue on the fused kernel's outputs: the dual residual
    RMSNorm alone (HBM-bound, GB/s against 8 TB/s), and the whole drop-in (one
    o_proj GEMM over both outputs + the norm), with the stacked GEMM alone and
    the reference's two GEMMs (one per output) timed beside it."""
    import torch
    import torch.nn.functional as F
    from ttcd_amd import epilogue, work as W

    B, T = o_t.shape[0], o_t.shape[1]
    Hd, eps = cfg["hidden"], cfg["norm_eps"]
    dev = o_t.device
    g = torch.Generator(device=dev).manual_seed(2)
    r = torch.randn(B, T, Hd, device=dev, dtype=torch.bfloat16, generator=g)
    a_t, a_s = (torch.randn(B, T, Hd, device=dev, dtype=torch.bfloat16, generator=g)
                for _ in range(2))
    w = (1.0 + 0.1 * torch.randn(Hd, device=dev, generator=g)).to(torch.bfloat16)
    D_in = o_t.shape[2] * o_t.shape[3]
    wo = (torch.randn(Hd, D_in, device=dev, generator=g) * D_in ** -0.5).to(torch.bfloat16)
    o_proj = torch.nn.Linear(D_in, Hd, bias=False, device=dev, dtype=torch.bfloat16)
    o_proj.weight.data.copy_(wo)
    norm = types.SimpleNamespace(weight=w, bias=None, eps=eps)
    ms_n = time_gpu(lambda: epilogue.dual_residual_rmsnorm(a_t, a_s, r, w, eps), 20, 3)
    nbytes = W.epilogue_bytes(B * T, Hd)
    gbps = nbytes / (ms_n * 1e-3) / 1e9
    ms_f = time_gpu(lambda: epilogue.fused_attn_epilogue(o_proj, norm, o_t, o_s, r), 20, 3)
    ot2, os2 = o_t.reshape(B, T, -1), o_s.reshape(B, T, -1)
    ms_g2 = time_gpu(lambda: (F.linear(ot2, wo), F.linear(os2, wo)), 20, 3)
    st = epilogue._stacked(ot2, os2)
    ms_g1 = time_gpu(lambda: F.linear(st, wo), 20, 3)
    # the reference's two fla launches: each reads attn and residual and writes
    # y and the residual sum
    ref_bytes = 2 * 4 * B * T * Hd * 2 + 2 * Hd * 2
    return {"shape": {"rows": B * T, "hidden": Hd, "o_proj_in": D_in}, "norm_eps": eps,
            "norm_ms": ms_n, "norm_GB_per_s": gbps, "norm_frac_of_hbm_peak": gbps / PEAK_HBM_GBPS,
            "norm_algorithmic_bytes": nbytes, "reference_norm_launches_bytes": ref_bytes,
            "drop_in_ms": ms_f, "stacked_gemm_ms": ms_g1, "two_gemms_ms": ms_g2}


def second_shape_measure(name: str, steps: int = 10, warmup: int = 3) -> dict:
    """The other BASELINE layer shape (config 3, SmolLM2-360M: Hq=15, Hkv=5,
    D=64) timed like the headline: the fused kernel with both LSEs, the two
    separate windowed calls, and the LSE variant; TFLOP/s over the teacher
    band."""
    import torch
    from ttcd_amd import fused_dual_window_attn, lse_dual_window_attn, window_attn, work as W

    cfg = CONFIGS[name]
    B, T, H, HK, D, wt, ws = (cfg[k] for k in ("B", "T", "Hq", "Hkv", "D", "wt", "ws"))
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, T, H, D, device=dev, dtype=torch.bfloat16, generator=gen)
    k = torch.randn(B, T, HK, D, device=dev, dtype=torch.bfloat16, generator=gen)
    v = torch.randn(B, T, HK, D, device=dev, dtype=torch.bfloat16, generator=gen)
    F, F_s = W.attn_flops(B, H, D, T, wt), W.attn_flops(B, H, D, T, ws)
    ms = time_gpu(lambda: fused_dual_window_attn(q, k, v, wt, ws, return_lse=True), steps, warmup)
    ms_two = time_gpu(lambda: (window_attn(q, k, v, wt), window_attn(q, k, v, ws)), steps, 2)
    ms_lse = time_gpu(lambda: lse_dual_window_attn(q, k, v, wt, ws), steps, 2)
    tf = F / (ms * 1e-3) / 1e12
    log(f"{name}: fused {ms:.3f} ms {tf:.0f} TF/s ({100 * tf / PEAK_BF16_TFLOPS:.1f}%), "
        f"two calls {ms_two:.3f} ms, LSE variant {ms_lse:.3f} ms")
    return {"workload": cfg["name"], "B": B, "T": T, "Hq": H, "Hkv": HK, "head_dim": D,
            "window_teacher": wt, "window_student": ws, "flops": F, "ms": ms, "tflops": tf,
            "frac_of_bf16_peak": tf / PEAK_BF16_TFLOPS, "tokens_per_s": B * T / (ms * 1e-3),
            "two_separate_calls_ms": ms_two, "fused_speedup_vs_two_calls": ms_two / ms,
            "ideal_speedup_vs_two_calls": (F + F_s) / F, "lse_variant_ms": ms_lse}


def source_hash(*names: str) -> str:
    """sha256 over the named kernel sources (ttcd_amd/csrc), to tie a profile
    measured on one build to the build being timed."""
    import hashlib
    h = hashlib.sha256()
    for n in names:
        with open(os.path.join(ROOT, "ttcd_amd", "csrc", n), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


ATTN_SOURCES = ("attn.hip", "schedule.h")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="qwen3", choices=sorted(CONFIGS))
    ap.add_argument("--no-extra", action="store_true", help="skip comparators and conv")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-numerics", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--seqlen", type=int, default=32768, help="prompt length of --only e2e")
    ap.add_argument("--only", choices=["fused", "band", "lse", "causal", "sdpa", "conv", "copy",
                                       "prologue", "epilogue", "sweep", "e2e"],
                    help="profiling mode: run one workload --steps times and print its timing")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the path is single-GPU; "
              "multi-GPU sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch
    from ttcd_amd import (causal_dwconv_x, fused_dual_window_attn, lse_dual_window_attn,
                          window_attn)
    from ttcd_amd import work as W

    if args.only == "e2e":
        with torch.inference_mode():
            print(json.dumps({"only": "e2e", **e2e_measure(args.steps, args.warmup,
                                                            T=args.seqlen, paths=("fused",))}),
                  flush=True)
        return 0
    if args.only == "sweep":
        with torch.inference_mode():
            print(json.dumps({"only": "sweep", "points": sweep_measure(args.steps, args.warmup)}),
                  flush=True)
        return 0
    if args.only:
        return profile_one(args)

    cfg = CONFIGS[args.config]
    B, T, H, HK, D, wt, ws = (cfg[k] for k in ("B", "T", "Hq", "Hkv", "D", "wt", "ws"))
    dev = torch.device("cuda:0")
    log(f"device {torch.cuda.get_device_name(dev)}; config {cfg}")
    gen = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, T, H, D, device=dev, dtype=torch.bfloat16, generator=gen)
    k = torch.randn(B, T, HK, D, device=dev, dtype=torch.bfloat16, generator=gen)
    v = torch.randn(B, T, HK, D, device=dev, dtype=torch.bfloat16, generator=gen)
    torch.cuda.synchronize()

    F = W.attn_flops(B, H, D, T, wt)
    F_s = W.attn_flops(B, H, D, T, ws)
    res = {}
    with torch.inference_mode():
        fused = lambda: fused_dual_window_attn(q, k, v, wt, ws, return_lse=True)  # noqa: E731
        ms = time_gpu(fused, args.steps, args.warmup)
        tflops = F / (ms * 1e-3) / 1e12
        log(f"fused dual-window: {ms:.3f} ms/step, {tflops:.1f} TFLOP/s "
            f"({100 * tflops / PEAK_BF16_TFLOPS:.1f}% of bf16 peak)")
        if not args.no_extra:
            two = lambda: (window_attn(q, k, v, wt), window_attn(q, k, v, ws))  # noqa: E731
            ms_two = time_gpu(two, max(3, args.steps // 2), 2)
            ms_t = time_gpu(lambda: window_attn(q, k, v, wt), max(3, args.steps // 2), 2)
            ms_lse = time_gpu(lambda: lse_dual_window_attn(q, k, v, wt, ws),
                              max(3, args.steps // 2), 2)
            ms_x = time_gpu(lambda: fused_dual_window_attn(q, k, v, wt, ws, return_lse=True,
                                                           exact_max=True),
                            max(3, args.steps // 2), 2)
            log(f"two calls {ms_two:.3f} ms, teacher-only {ms_t:.3f} ms, LSE variant {ms_lse:.3f} ms, "
                f"fused with the exact running max {ms_x:.3f} ms")
            res["comparators"] = {
                "two_separate_calls_ms": ms_two,
                "fused_speedup_vs_two_calls": ms_two / ms,
                "ideal_speedup_vs_two_calls": (F + F_s) / F,
                "teacher_only_call_ms": ms_t,
                "teacher_only_call_tflops": F / (ms_t * 1e-3) / 1e12,
                "lse_variant_ms": ms_lse,
                "comparator": "own gfx950 single-band kernel called at w_T then w_S",
                # exact_max=True: the reference kernel's exact running max (numerics_config1
                # reports how many outputs then match its emulation bit for bit)
                "fused_exact_max_ms": ms_x,
                "fused_exact_max_tflops": F / (ms_x * 1e-3) / 1e12,
            }
            del two
            # conv at the reference's benchmark shape (profiling/fused_conv.py:77)
            xg = torch.Generator(device=dev).manual_seed(0)
            x = torch.randn(1, 16, 4096, 3072, device=dev, dtype=torch.bfloat16, generator=xg)
            w = torch.randn(3072, 5, device=dev, dtype=torch.bfloat16, generator=xg)
            ms_c = time_gpu(lambda: causal_dwconv_x(x, w), 20, 3)
            nbytes = W.conv_bytes(16, 4096, 3072, 5)
            gbps = nbytes / (ms_c * 1e-3) / 1e9
            log(f"conv (1,16,4096,3072) K=5: {ms_c:.4f} ms, {gbps:.0f} GB/s")
            res["conv"] = {"shape": [1, 16, 4096, 3072], "K": 5, "ms": ms_c, "GB_per_s": gbps,
                           "frac_of_hbm_peak": gbps / PEAK_HBM_GBPS,
                           "algorithmic_bytes": nbytes}
            del x, w
            res["prologue"] = prologue_measure(q, k, cfg)
            log(f"prologue (q/k RMSNorm + rotary): {res['prologue']}")
            o_t, o_s = fused_dual_window_attn(q, k, v, wt, ws)
            res["epilogue"] = epilogue_measure(o_t, o_s, cfg)
            log(f"epilogue (o_proj + dual residual RMSNorm): {res['epilogue']}")
            del o_t, o_s
            if args.config == "qwen3":
                res["recipes_64k"] = recipes_measure(q, k, v)
                res["second_kernel_agreement"] = second_kernel_agreement(q, k, v, wt, ws)
                log(f"fused vs single-band kernel, every row: {res['second_kernel_agreement']}")
                res["vendor_sdpa_full_causal"] = vendor_sdpa_measure(q, k, v)
                res["smollm2"] = second_shape_measure("smollm2")
            res["config4_sweep"] = sweep_measure()
            res["e2e_prefill"] = e2e_measure()
            # the length the reference's end-to-end numbers are quoted at
            e64 = e2e_measure(steps=3, warmup=1, T=65536, paths=("fused", "stock"))
            e64["reference_h100_ms"] = {
                "ipttcdv9_unpatched": 629.0, "ipttcdv9_fused_attn_triton_conv": 526.1,
                "hardware": "one H100 80GB", "source": "profiling/REPORT.md:25, :321",
                "note": "other hardware and the reference's generate() prefill; context only"}
            res["e2e_prefill_64k"] = e64
            e64c = e2e_chunked_measure()
            e64c["one_shot_fused_ms"] = e64["fused"]["ms"]
            e64c["vs_one_shot"] = e64["fused"]["ms"] / e64c["ms"]
            res["e2e_prefill_64k_chunked"] = e64c
    # HBM bytes per launch measured by rocprofv3 (FETCH_SIZE / WRITE_SIZE) on
    # the build whose attention sources hash to `attn_sources_sha256`; dropped
    # (null) when the sources timed here differ
    traffic, traffic_note = None, "no HBM-traffic profile for this config"
    tpath = os.path.join(ROOT, "profiles", f"hbm_traffic_{args.config}.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
        if tj.get("attn_sources_sha256") == source_hash(*ATTN_SOURCES):
            traffic = tj.get("fused_dual_window_attn_bytes_per_launch")
            traffic_note = f"rocprofv3 FETCH_SIZE/WRITE_SIZE, {os.path.basename(tpath)}"
        else:
            traffic_note = "stale: profile measured on other attention sources"

    out = {
        "metric": METRIC,
        "value": tflops,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: q/k/v bf16 N(0,1), seed 0, resident in HBM",
        "config": {"workload": f"dual-window attention prefill, {cfg['name']}", "B": B, "T": T,
                   "Hq": H, "Hkv": HK, "head_dim": D, "window_teacher": wt,
                   "window_student": ws, "outputs": "o_teacher, o_student, lse_teacher, lse_student"},
        "pct_bf16_peak": 100 * tflops / PEAK_BF16_TFLOPS,
        "tokens_per_s": B * T / (ms * 1e-3),
        "flops_per_step": F,
        # secondary line: the work of the two separate calls the fused call
        # replaces (teacher band + student band), over the same time
        "two_call_equivalent_flops": F + F_s,
        "two_call_equivalent_tflops": (F + F_s) / (ms * 1e-3) / 1e12,
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": tflops / PEAK_BF16_TFLOPS, "traffic": traffic,
                     "traffic_source": traffic_note},
        **res,
    }
    # The CPU leg: the reference's CPU path (restated in oracle/), timed as the
    # cpu_baseline and used as the checker of the config-1 numerics. No other
    # part of this file touches oracle/.
    if not args.no_cpu:
        log("CPU baseline ...")
        out["cpu_baseline"] = cpu_baseline(q, k, v, cfg, args.cpu_seconds)
        log(f"cpu_baseline: {out['cpu_baseline']['value']:.4f} TFLOP/s "
            f"on {out['cpu_baseline']['cores']} threads")
        if not args.no_numerics:
            out["numerics_config1"] = numerics_report()
            log(f"numerics: {out['numerics_config1']}")
            out["numerics_config1_d128"] = numerics_report(128)
            log(f"numerics at D=128: {out['numerics_config1_d128']}")
            if args.config == "qwen3":
                with torch.inference_mode():
                    out["numerics_headline"] = numerics_headline(q, k, v, wt, ws)
                log(f"numerics at the headline shape: {out['numerics_headline']}")
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
