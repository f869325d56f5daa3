// conv.hip - chunk-local causal depthwise conv on the (N, C, D) layout for
// gfx950. Replaces the Triton kernel _causal_dwconv_fwd
// (profiling/fused_conv.py:24-48): y[n,c,d] = sum_j w[d,j] * x[n,c-(K-1)+j,d]
// with left zero padding inside each chunk, fp32 accumulation in tap order
// j = 0..K-1 (acc = fma(x, w, acc) from acc = +0), one RNE rounding to the
// input dtype.
//
// The op is HBM-bound (one read of x, one write of y), so there is no MFMA
// here. Each thread owns 16 bytes along D (8 bf16 channels) and a run of R
// consecutive rows along C: consecutive lanes own consecutive 16-byte
// chunks, so every row access of a wavefront is one fully coalesced 1 KiB
// transaction. The K-1 previous rows stay in registers as a sliding window,
// so x is fetched once per row plus a K-1 row halo per run (the halo misses
// L2 as often as not: it is requested while the neighbouring run fetches the
// same rows, so HBM reads are (R + K - 1) / R of x). y is written with
// non-temporal stores: it is consumed by the next op, not by this kernel.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "internal.h"

namespace ttcd {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename X>
struct Cvt;
template <>
struct Cvt<__bf16> {
  __device__ static float to_f(__bf16 v) { return static_cast<float>(v); }
  __device__ static __bf16 from_f(float v) { return static_cast<__bf16>(v); }
};
template <>
struct Cvt<_Float16> {
  __device__ static float to_f(_Float16 v) { return static_cast<float>(v); }
  // The empty asm pins the fp32 sum in a register first. Without it the compiler
  // fuses the last tap's fma with this conversion (v_fma_mix{lo,hi}_f16), which
  // rounds once from the exact value instead of fp32-then-fp16 as the reference
  // conv does, and about one output in 8K differs in its last bit.
  __device__ static _Float16 from_f(float v) {
    __asm__("" : "+v"(v));
    return static_cast<_Float16>(v);
  }
};
template <>
struct Cvt<float> {
  __device__ static float to_f(float v) { return v; }
  __device__ static float from_f(float v) { return v; }
};

template <typename X>
union Pack16 {
  static constexpr int N = 16 / sizeof(X);
  u32x4 raw;
  X e[N];
};

constexpr int kRows = 16;  // rows of C per thread

template <typename X, typename W, int K>
__global__ __launch_bounds__(256) void dwconv_vec_kernel(const X* __restrict__ x,
                                                         const W* __restrict__ w,
                                                         X* __restrict__ y, int64_t N, int C,
                                                         int D, int nseg) {
  constexpr int V = Pack16<X>::N;
  const int ngroups = D / V;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = N * nseg * (int64_t)ngroups;
  if (gid >= total) return;
  const int dg = (int)(gid % ngroups);
  const int64_t rest = gid / ngroups;
  const int seg = (int)(rest % nseg);
  const int64_t n = rest / nseg;
  const int d0 = dg * V;
  const int c0 = seg * kRows;

  float wr[K][V];
#pragma unroll
  for (int e = 0; e < V; ++e)
#pragma unroll
    for (int j = 0; j < K; ++j) wr[j][e] = Cvt<W>::to_f(w[(int64_t)(d0 + e) * K + j]);

  const X* xb = x + n * C * (int64_t)D + d0;
  X* yb = y + n * C * (int64_t)D + d0;

  // win[t] holds row c - (K-1) + t for the row c being produced.
  float win[K][V];
#pragma unroll
  for (int t = 0; t < K - 1; ++t) {
    const int c = c0 - (K - 1) + t;
    Pack16<X> p;
    p.raw = u32x4{0u, 0u, 0u, 0u};
    if (c >= 0) p.raw = *reinterpret_cast<const u32x4*>(xb + (int64_t)c * D);
#pragma unroll
    for (int e = 0; e < V; ++e) win[t][e] = Cvt<X>::to_f(p.e[e]);
  }

  const int rows = min(kRows, C - c0);
  if (rows == kRows) {
    Pack16<X> in[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
      in[r].raw = *reinterpret_cast<const u32x4*>(xb + (int64_t)(c0 + r) * D);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
#pragma unroll
      for (int e = 0; e < V; ++e) win[K - 1][e] = Cvt<X>::to_f(in[r].e[e]);
      Pack16<X> out;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < K; ++j) acc = fmaf(win[j][e], wr[j][e], acc);
        out.e[e] = Cvt<X>::from_f(acc);
      }
      __builtin_nontemporal_store(out.raw, reinterpret_cast<u32x4*>(yb + (int64_t)(c0 + r) * D));
#pragma unroll
      for (int t = 0; t < K - 1; ++t)
#pragma unroll
        for (int e = 0; e < V; ++e) win[t][e] = win[t + 1][e];
    }
  } else {
    for (int r = 0; r < rows; ++r) {
      Pack16<X> in;
      in.raw = *reinterpret_cast<const u32x4*>(xb + (int64_t)(c0 + r) * D);
#pragma unroll
      for (int e = 0; e < V; ++e) win[K - 1][e] = Cvt<X>::to_f(in.e[e]);
      Pack16<X> out;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < K; ++j) acc = fmaf(win[j][e], wr[j][e], acc);
        out.e[e] = Cvt<X>::from_f(acc);
      }
      *reinterpret_cast<u32x4*>(yb + (int64_t)(c0 + r) * D) = out.raw;
#pragma unroll
      for (int t = 0; t < K - 1; ++t)
#pragma unroll
        for (int e = 0; e < V; ++e) win[t][e] = win[t + 1][e];
    }
  }
}

// Any K (<= 64), any D: one thread per output element, taps re-read through
// the cache. Same fixed accumulation order as the vector kernel.
template <typename X, typename W>
__global__ __launch_bounds__(256) void dwconv_scalar_kernel(const X* __restrict__ x,
                                                            const W* __restrict__ w,
                                                            X* __restrict__ y, int64_t N, int C,
                                                            int D, int K) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = N * C * (int64_t)D;
  if (gid >= total) return;
  const int d = (int)(gid % D);
  const int64_t rest = gid / D;
  const int c = (int)(rest % C);
  const int64_t n = rest / C;
  const X* xb = x + n * C * (int64_t)D + d;
  float acc = 0.f;
  for (int j = 0; j < K; ++j) {
    const int src = c - (K - 1) + j;
    const float xv = src >= 0 ? Cvt<X>::to_f(xb[(int64_t)src * D]) : 0.f;
    acc = fmaf(xv, Cvt<W>::to_f(w[(int64_t)d * K + j]), acc);
  }
  y[gid] = Cvt<X>::from_f(acc);
}

template <typename X, typename W, int K>
hipError_t launch_vec(const void* x, const void* w, void* y, int64_t N, int C, int D,
                      hipStream_t st) {
  constexpr int V = Pack16<X>::N;
  const int nseg = (C + kRows - 1) / kRows;
  const int64_t total = N * nseg * (int64_t)(D / V);
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL((dwconv_vec_kernel<X, W, K>), dim3((unsigned)blocks), dim3(256), 0, st,
                     static_cast<const X*>(x), static_cast<const W*>(w), static_cast<X*>(y), N,
                     C, D, nseg);
  return hipGetLastError();
}

template <typename X, typename W>
hipError_t launch_typed(const void* x, const void* w, void* y, int64_t N, int C, int D, int K,
                        hipStream_t st) {
  constexpr int V = Pack16<X>::N;
  const bool vec_ok = (D % V) == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0 &&
                      (reinterpret_cast<uintptr_t>(y) % 16) == 0;
  if (vec_ok) {
    switch (K) {
      case 1: return launch_vec<X, W, 1>(x, w, y, N, C, D, st);
      case 2: return launch_vec<X, W, 2>(x, w, y, N, C, D, st);
      case 3: return launch_vec<X, W, 3>(x, w, y, N, C, D, st);
      case 4: return launch_vec<X, W, 4>(x, w, y, N, C, D, st);
      case 5: return launch_vec<X, W, 5>(x, w, y, N, C, D, st);
      case 6: return launch_vec<X, W, 6>(x, w, y, N, C, D, st);
      case 7: return launch_vec<X, W, 7>(x, w, y, N, C, D, st);
      case 8: return launch_vec<X, W, 8>(x, w, y, N, C, D, st);
      default: break;
    }
  }
  const int64_t total = N * C * (int64_t)D;
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL((dwconv_scalar_kernel<X, W>), dim3((unsigned)blocks), dim3(256), 0, st,
                     static_cast<const X*>(x), static_cast<const W*>(w), static_cast<X*>(y), N,
                     C, D, K);
  return hipGetLastError();
}

template <typename X>
hipError_t launch_w(const void* x, const void* w, void* y, int64_t N, int C, int D, int K,
                    Elem wt, hipStream_t st) {
  switch (wt) {
    case Elem::BF16: return launch_typed<X, __bf16>(x, w, y, N, C, D, K, st);
    case Elem::F16: return launch_typed<X, _Float16>(x, w, y, N, C, D, K, st);
    default: return launch_typed<X, float>(x, w, y, N, C, D, K, st);
  }
}

}  // namespace

hipError_t launch_dwconv(const void* x, const void* w, void* y, int64_t N, int C, int D, int K,
                         Elem xt, Elem wt, hipStream_t stream) {
  switch (xt) {
    case Elem::BF16: return launch_w<__bf16>(x, w, y, N, C, D, K, wt, stream);
    case Elem::F16: return launch_w<_Float16>(x, w, y, N, C, D, K, wt, stream);
    default: return launch_w<float>(x, w, y, N, C, D, K, wt, stream);
  }
}

}  // namespace ttcd
