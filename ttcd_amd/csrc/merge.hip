// merge.hip - exact log-sum-exp merge of two attention partials over
// disjoint key sets (the ring-attention identity), gfx950.
// Replaces _lse_merge_kernel and the o_t[:, :WS] = o_s[:, :WS] copy of
// lse_dual_window_attn_fa3_fast (profiling/lse_dual_attn.py:106-131,
// :151-159):
//   m  = max(ls, lf); lt = m + log(exp(ls-m) + exp(lf-m))
//   o_t = o_s * exp(ls-lt) + o_f * exp(lf-lt)         (fp32, one rounding)
// Rows before row_start, and rows whose far partial is empty (lf = -inf),
// are copied from o_s bit for bit. HBM-bound elementwise pass: each thread
// moves 16 bytes of each operand with coalesced vector accesses.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "internal.h"

namespace ttcd {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
union P8 {
  u32x4 raw;
  T e[8];
};

template <typename T>
__global__ __launch_bounds__(256) void lse_merge_kernel(const T* __restrict__ os,
                                                        const float* __restrict__ ls,
                                                        const T* __restrict__ of,
                                                        const float* __restrict__ lf,
                                                        T* __restrict__ ot, int B, int T_, int H,
                                                        int D, int row_start, int64_t sb,
                                                        int64_t st, int64_t sh) {
  const int ng = D / 8;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)B * T_ * H * ng;
  if (gid >= total) return;
  const int dg = (int)(gid % ng);
  int64_t rest = gid / ng;
  const int h = (int)(rest % H);
  rest /= H;
  const int t = (int)(rest % T_);
  const int b = (int)(rest / T_);
  const int64_t off = b * sb + t * st + h * sh + dg * 8;
  P8<T> s;
  s.raw = *reinterpret_cast<const u32x4*>(os + off);
  if (t < row_start) {
    *reinterpret_cast<u32x4*>(ot + off) = s.raw;
    return;
  }
  const int64_t li = ((int64_t)b * H + h) * T_ + t;
  const float a = ls[li], f = lf[li];
  if (f == -INFINITY) {
    *reinterpret_cast<u32x4*>(ot + off) = s.raw;
    return;
  }
  float wa, wf;
  if (a == -INFINITY) {
    wa = 0.f;
    wf = 1.f;
  } else {
    const float mx = fmaxf(a, f);
    const float lt = mx + logf(expf(a - mx) + expf(f - mx));
    wa = expf(a - lt);
    wf = expf(f - lt);
  }
  P8<T> fv, out;
  fv.raw = *reinterpret_cast<const u32x4*>(of + off);
#pragma unroll
  for (int e = 0; e < 8; ++e)
    out.e[e] = static_cast<T>(fmaf(static_cast<float>(fv.e[e]), wf, static_cast<float>(s.e[e]) * wa));
  *reinterpret_cast<u32x4*>(ot + off) = out.raw;
}

template <typename T>
hipError_t launch_typed(const void* o_s, const float* lse_s, const void* o_f,
                        const float* lse_f, void* o_t, int B, int T_, int H, int D,
                        int row_start, int64_t sb, int64_t st, int64_t sh, hipStream_t stream) {
  const int64_t total = (int64_t)B * T_ * H * (D / 8);
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL((lse_merge_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const T*>(o_s), lse_s, static_cast<const T*>(o_f), lse_f,
                     static_cast<T*>(o_t), B, T_, H, D, row_start, sb, st, sh);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_lse_merge(const void* o_s, const float* lse_s, const void* o_f,
                            const float* lse_f, void* o_t, int B, int T, int H, int D,
                            int row_start, int64_t sb, int64_t st, int64_t sh, Elem dtype,
                            hipStream_t stream) {
  if (dtype == Elem::BF16)
    return launch_typed<__bf16>(o_s, lse_s, o_f, lse_f, o_t, B, T, H, D, row_start, sb, st, sh,
                                stream);
  return launch_typed<_Float16>(o_s, lse_s, o_f, lse_f, o_t, B, T, H, D, row_start, sb, st, sh,
                                stream);
}

}  // namespace ttcd
