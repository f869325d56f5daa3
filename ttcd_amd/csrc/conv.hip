// conv.hip - chunk-local causal depthwise conv on the (N, C, D) layout for
// gfx950. Replaces the Triton kernel _causal_dwconv_fwd
// (profiling/fused_conv.py:24-48): y[n,c,d] = sum_j w[d,j] * x[n,c-(K-1)+j,d]
// with left zero padding inside each chunk, fp32 accumulation in tap order
// j = 0..K-1 (acc = fma(x, w, acc) from acc = +0), one RNE rounding to the
// input dtype.
//
// The op is HBM-bound (one read of x, one write of y), so there is no MFMA
// here. Each thread owns 16 bytes along D (8 bf16 channels) and a run of R
// consecutive rows along C, and the K-1 previous rows stay in registers as a
// sliding window. For K <= 8 (dwconv_halo_kernel) a wavefront holds 16
// groups along D of 4 consecutive runs, and each run's K-1 halo rows come
// from the run below it through a lane shuffle, so x is read (4R + K - 1) /
// 4R times. (A halo re-read from memory by every run misses L2 as often as
// not: it is requested while the neighbouring run fetches the same rows,
// which cost 25 % more HBM reads at R = 16.) y is written with non-temporal
// stores: it is consumed by the next op, not by this kernel. Other K, or
// unaligned tensors, take dwconv_scalar_kernel.
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

// Shared-halo layout (K <= kRows + 1): a wavefront owns 16 consecutive
// 16-byte groups along D (lane % 16) of 4 consecutive runs along C (lane /
// 16), so each row access is four contiguous 256-byte pieces. The K-1 halo
// rows of run g are the last rows of run g-1, taken from the lanes 16 below
// with a lane shuffle; only the first run of a wavefront reads its halo from
// memory, so x is read (kRows * 4 + K - 1) / (kRows * 4) times instead of
// (kRows + K - 1) / kRows.
template <typename X, typename W, int K>
__global__ __launch_bounds__(256) void dwconv_halo_kernel(const X* __restrict__ x,
                                                          const W* __restrict__ w,
                                                          X* __restrict__ y, int64_t N, int C,
                                                          int D, int nseg) {
  static_assert(K - 1 <= kRows, "the halo must lie within the previous run");
  constexpr int V = Pack16<X>::N;
  const int ngroups = D / V;
  const int ntile = (ngroups + 15) / 16;
  const int nquad = (nseg + 3) / 4;
  const int lane = threadIdx.x & 63;
  // one wavefront per (n, quad of runs, 16-group tile); whole wavefronts leave
  const int64_t wid = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t total = N * nquad * (int64_t)ntile;
  if (wid >= total) return;
  const int tile = (int)(wid % ntile);
  const int64_t rest = wid / ntile;
  const int quad = (int)(rest % nquad);
  const int64_t n = rest / nquad;
  const int g = lane >> 4;
  const int dg = tile * 16 + (lane & 15);
  const bool col_ok = dg < ngroups;
  const int d0 = (col_ok ? dg : 0) * V;  // idle lanes read a valid group, store nothing
  const int c0 = (quad * 4 + g) * kRows;
  const int rows = col_ok ? max(0, min(kRows, C - c0)) : 0;

  float wr[K][V];
#pragma unroll
  for (int e = 0; e < V; ++e)
#pragma unroll
    for (int j = 0; j < K; ++j) wr[j][e] = Cvt<W>::to_f(w[(int64_t)(d0 + e) * K + j]);

  const X* xb = x + n * C * (int64_t)D + d0;
  X* yb = y + n * C * (int64_t)D + d0;

  Pack16<X> in[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    in[r].raw = u32x4{0u, 0u, 0u, 0u};
    if (r < rows) in[r].raw = *reinterpret_cast<const u32x4*>(xb + (int64_t)(c0 + r) * D);
  }

  // win[t] holds row c - (K-1) + t for the row c being produced. Every lane
  // takes part in the shuffles; run g > 0 has a full run g-1 below it.
  float win[K][V];
#pragma unroll
  for (int t = 0; t < K - 1; ++t) {
    Pack16<X> p;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      p.raw[q] = (uint32_t)__shfl_up((int)in[kRows - (K - 1) + t].raw[q], 16, 64);
    if (g == 0) {
      const int c = c0 - (K - 1) + t;
      p.raw = u32x4{0u, 0u, 0u, 0u};
      if (c >= 0 && rows > 0) p.raw = *reinterpret_cast<const u32x4*>(xb + (int64_t)c * D);
    }
#pragma unroll
    for (int e = 0; e < V; ++e) win[t][e] = Cvt<X>::to_f(p.e[e]);
  }

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
    if (r < rows)
      __builtin_nontemporal_store(out.raw, reinterpret_cast<u32x4*>(yb + (int64_t)(c0 + r) * D));
#pragma unroll
    for (int t = 0; t < K - 1; ++t)
#pragma unroll
      for (int e = 0; e < V; ++e) win[t][e] = win[t + 1][e];
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
  const int64_t waves = N * ((nseg + 3) / 4) * (int64_t)((D / V + 15) / 16);
  const int64_t blocks = (waves * 64 + 255) / 256;
  hipLaunchKernelGGL((dwconv_halo_kernel<X, W, K>), dim3((unsigned)blocks), dim3(256), 0, st,
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
