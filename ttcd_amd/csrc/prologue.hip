// prologue.hip - attention prologue for gfx950: per-head RMSNorm of q and k
// (qk_norm) fused with the rotary embedding, one pass over q and k.
//
// Replaces, at the call site profiling/patches.py:254-268 (also
// custom_models/ipttcd/modeling_ipttcdv9.py:728-738), the four launches
//   q, k = attn.q_norm(q), attn.k_norm(k)      fla/modules/layernorm.py:189-251
//   q, k = attn.rotary(q, k, seqlen_offset=..) fla/modules/rotary.py:43-135
// which each read and write all of q or k. Numerics per row of D elements:
//   RMSNorm (IS_RMS_NORM, HAS_WEIGHT): x in fp32, var = sum(x*x) / D,
//     rstd = 1 / sqrt(var + eps), y = (x * rstd) * w, rounded to the input
//     dtype (layernorm.py:219-251);
//   rotary, GPT-NeoX halves (INTERLEAVED = False): with x0 = y[:D/2],
//     x1 = y[D/2:] and the dtype-rounded cos/sin tables at position t + offset,
//     o0 = x0*cos - x1*sin, o1 = x0*sin + x1*cos in fp32, rounded to the input
//     dtype (rotary.py:93-107). Both products are products of two 16-bit
//     values, exact in fp32, so every o is the correctly rounded fp32 value
//     whatever the evaluation order.
// The only freedom left is the order of the sum of squares (here: each lane
// sums its 16 squares in element order, then a butterfly over the row's lanes).
//
// Layout: lane `sub` of a row owns the 8 element pairs (d, d + D/2) for
// d = 8*sub .. 8*sub+7, so the rotation is lane-local; a row spans D/16 lanes
// and a wavefront handles 64 / (D/16) rows per step. Rows run over all q rows
// (b, t, h) and then all k rows; consecutive rows of one token are
// consecutive in memory, so every access of a wavefront is coalesced. The
// cos/sin rows of a token are shared by all its heads (L1/L2 hits); q and k
// are read once, with non-temporal loads. The outputs are stored normally:
// non-temporal stores measure 11 % faster for this kernel alone but make the
// attention kernel that reads them next fetch them from HBM rather than the
// 256 MiB last-level cache (the whole prefill 0.2-0.7 % slower at 32K).
//
// rope_table_kernel builds those tables as the reference does
// (rotary.py:441-490 with pos_idx_in_fp32): freq = fp32(t) * inv_freq[i]
// (one fp32 rounding, torch.outer), cos / sin of that fp32 value, rounded to
// the dtype.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "internal.h"

namespace ttcd {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
union V8 {
  u32x4 raw;
  T e[8];
};

template <typename W>
__device__ __forceinline__ float to_f(W v) {
  return static_cast<float>(v);
}

// An fp32 value rounded to T as a separate step, as the reference stores an
// fp32 result: without the opaque copy the compiler fuses the last fma and
// the conversion into v_fma_mix{lo,hi}_f16, which rounds the exact value
// once, straight to f16, instead of to fp32 and then to f16.
template <typename T>
__device__ __forceinline__ T round_to(float v) {
  asm volatile("" : "+v"(v));
  return static_cast<T>(v);
}

// Rows per lane: their loads are all issued before the first is used. One
// row at D = 128 and two at D = 64 measured fastest (5 % and 8 % below four
// rows taken one after another; four or more rows in flight at once ran
// slower at D = 128).
constexpr int prologue_steps(int D) { return D == 128 ? 1 : 2; }

template <typename T, typename W, int D, bool NORM>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(PrologueArgs a) {
  constexpr int R = D / 2;    // rotary pairs per row
  constexpr int L = D / 16;   // lanes per row
  constexpr int RPW = 64 / L;  // rows per wavefront step
  constexpr int ITER = prologue_steps(D);  // rows per lane
  const int lane = threadIdx.x & 63;
  const int sub = lane % L;
  const int rw = lane / L;
  const int d0 = 8 * sub;

  float wq[2][8], wk[2][8];
  if (NORM) {
    const W* qw = static_cast<const W*>(a.q_w);
    const W* kw = static_cast<const W*>(a.k_w);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      wq[0][e] = to_f(qw[d0 + e]);
      wq[1][e] = to_f(qw[R + d0 + e]);
      wk[0][e] = to_f(kw[d0 + e]);
      wk[1][e] = to_f(kw[R + d0 + e]);
    }
  }

  const int64_t rows_q = (int64_t)a.B * a.T * a.Hq;
  const int64_t rows = rows_q + (int64_t)a.B * a.T * a.Hkv;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / 64;
  // every step's loads are issued before any step is computed, so ITER rows
  // per lane are in flight at once
  V8<T> x0[ITER], x1[ITER], c[ITER], s[ITER];
  T* dst[ITER];
  bool valid[ITER], isk[ITER];
#pragma unroll
  for (int it = 0; it < ITER; ++it) {
    const int64_t r = (wave * ITER + it) * RPW + rw;
    valid[it] = r < rows;
    const bool is_k = r >= rows_q;
    isk[it] = is_k;
    const int64_t rr = valid[it] ? (is_k ? r - rows_q : r) : 0;
    const int H = is_k ? a.Hkv : a.Hq;
    const int h = (int)(rr % H);
    const int64_t bt = rr / H;
    const int t = (int)(bt % a.T);
    const int b = (int)(bt / a.T);
    const T* src = is_k ? static_cast<const T*>(a.k) + b * a.k_sb + t * a.k_st + h * a.k_sh
                        : static_cast<const T*>(a.q) + b * a.q_sb + t * a.q_st + h * a.q_sh;
    dst[it] = is_k ? static_cast<T*>(a.k_out) + b * a.ko_sb + t * a.ko_st + h * a.ko_sh
                   : static_cast<T*>(a.q_out) + b * a.qo_sb + t * a.qo_st + h * a.qo_sh;
    x0[it].raw = x1[it].raw = u32x4{0u, 0u, 0u, 0u};
    c[it].raw = s[it].raw = u32x4{0u, 0u, 0u, 0u};
    if (valid[it]) {
      x0[it].raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + d0));
      x1[it].raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + R + d0));
      const int64_t pos = (int64_t)t + a.offset;
      c[it].raw = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.cos) + pos * R + d0);
      s[it].raw = *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.sin) + pos * R + d0);
    }
  }
#pragma unroll
  for (int it = 0; it < ITER; ++it) {
    const bool is_k = isk[it];
    float y0[8], y1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      y0[e] = to_f(x0[it].e[e]);
      y1[e] = to_f(x1[it].e[e]);
    }
    if (NORM) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(y0[e], y0[e], ss);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(y1[e], y1[e], ss);
#pragma unroll
      for (int m = 1; m < L; m <<= 1) ss += __shfl_xor(ss, m, 64);
      const float rstd = 1.0f / sqrtf(ss / (float)D + a.eps);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // (x * rstd) * w, rounded to the input dtype as the norm's output is
        y0[e] = to_f(round_to<T>((y0[e] * rstd) * (is_k ? wk[0][e] : wq[0][e])));
        y1[e] = to_f(round_to<T>((y1[e] * rstd) * (is_k ? wk[1][e] : wq[1][e])));
      }
    }
    V8<T> o0, o1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float ce = to_f(c[it].e[e]), se = to_f(s[it].e[e]);
      o0.e[e] = round_to<T>(y0[e] * ce - y1[e] * se);
      o1.e[e] = round_to<T>(y0[e] * se + y1[e] * ce);
    }
    if (valid[it]) {
      *reinterpret_cast<u32x4*>(dst[it] + d0) = o0.raw;
      *reinterpret_cast<u32x4*>(dst[it] + R + d0) = o1.raw;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void rope_table_kernel(T* cos_t, T* sin_t, const float* inv_freq,
                                                         int rows, int half) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)rows * half) return;
  const int t = (int)(i / half);
  const int j = (int)(i % half);
  const float f = (float)t * inv_freq[j];
  cos_t[i] = static_cast<T>(cosf(f));
  sin_t[i] = static_cast<T>(sinf(f));
}

template <typename T, typename W, int D>
hipError_t launch_nr(const PrologueArgs& a, hipStream_t st) {
  constexpr int L = D / 16, RPW = 64 / L, ITER = prologue_steps(D);
  const int64_t rows = (int64_t)a.B * a.T * (a.Hq + a.Hkv);
  const int64_t waves = (rows + (int64_t)RPW * ITER - 1) / ((int64_t)RPW * ITER);
  const int64_t blocks = (waves + 3) / 4;
  if (a.q_w != nullptr) {
    hipLaunchKernelGGL((qk_norm_rope_kernel<T, W, D, true>), dim3((unsigned)blocks), dim3(256), 0,
                       st, a);
  } else {
    hipLaunchKernelGGL((qk_norm_rope_kernel<T, W, D, false>), dim3((unsigned)blocks), dim3(256),
                       0, st, a);
  }
  return hipGetLastError();
}

template <typename T, typename W>
hipError_t launch_d(const PrologueArgs& a, hipStream_t st) {
  return a.D == 128 ? launch_nr<T, W, 128>(a, st) : launch_nr<T, W, 64>(a, st);
}

template <typename T>
hipError_t launch_w(const PrologueArgs& a, Elem wt, hipStream_t st) {
  switch (wt) {
    case Elem::BF16: return launch_d<T, __bf16>(a, st);
    case Elem::F16: return launch_d<T, _Float16>(a, st);
    default: return launch_d<T, float>(a, st);
  }
}

}  // namespace

hipError_t launch_qk_norm_rope(const PrologueArgs& a, Elem dtype, Elem wt, hipStream_t stream) {
  return dtype == Elem::BF16 ? launch_w<__bf16>(a, wt, stream) : launch_w<_Float16>(a, wt, stream);
}

hipError_t launch_rope_table(void* cos_t, void* sin_t, const float* inv_freq, int rows, int half,
                             Elem dtype, hipStream_t stream) {
  const int64_t n = (int64_t)rows * half;
  const unsigned blocks = (unsigned)((n + 255) / 256);
  if (dtype == Elem::BF16) {
    hipLaunchKernelGGL(rope_table_kernel<__bf16>, dim3(blocks), dim3(256), 0, stream,
                       static_cast<__bf16*>(cos_t), static_cast<__bf16*>(sin_t), inv_freq, rows,
                       half);
  } else {
    hipLaunchKernelGGL(rope_table_kernel<_Float16>, dim3(blocks), dim3(256), 0, stream,
                       static_cast<_Float16*>(cos_t), static_cast<_Float16*>(sin_t), inv_freq,
                       rows, half);
  }
  return hipGetLastError();
}

}  // namespace ttcd
