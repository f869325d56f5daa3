// merge.hip - exact log-sum-exp merge of two attention partials over
// disjoint key sets (the ring-attention identity), gfx950.
// Replaces _lse_merge_kernel and the o_t[:, :WS] = o_s[:, :WS] copy of
// lse_dual_window_attn_fa3_fast (profiling/lse_dual_attn.py:106-131,
// :151-159):
//   m  = max(ls, lf); lt = m + log(exp(ls-m) + exp(lf-m))
//   o_t = o_s * exp(ls-lt) + o_f * exp(lf-lt)         (fp32, one rounding)
// Rows before row_start, and rows whose far partial is empty (lf = -inf),
// are copied from o_s bit for bit. o_s and o_t share strides; o_f has its
// own (the LSE variant keeps it in a chunk-sized scratch). HBM-bound
// elementwise pass: each thread moves 16 bytes of each operand with
// coalesced vector accesses, non-temporal loads for the partials (read once).
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
__global__ __launch_bounds__(256) void lse_merge_kernel(MergeArgs a) {
  const T* __restrict__ os = static_cast<const T*>(a.o_s);
  const T* __restrict__ of = static_cast<const T*>(a.o_f);
  T* __restrict__ ot = static_cast<T*>(a.o_t);
  const int ng = a.D / 8;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.B * a.T * a.H * ng;
  if (gid >= total) return;
  const int dg = (int)(gid % ng);
  int64_t rest = gid / ng;
  const int h = (int)(rest % a.H);
  rest /= a.H;
  const int t = (int)(rest % a.T);
  const int b = (int)(rest / a.T);
  const int64_t off = b * a.sb + t * a.st + h * a.sh + dg * 8;
  P8<T> s;
  s.raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(os + off));
  if (t < a.row_start) {
    *reinterpret_cast<u32x4*>(ot + off) = s.raw;
    return;
  }
  const int64_t li = ((int64_t)b * a.H + h) * a.T + t;
  const float ls = a.lse_s[li], lf = a.lse_f[li];
  if (lf == -INFINITY) {
    *reinterpret_cast<u32x4*>(ot + off) = s.raw;
    return;
  }
  float wa, wf;
  if (ls == -INFINITY) {
    wa = 0.f;
    wf = 1.f;
  } else {
    const float mx = fmaxf(ls, lf);
    const float lt = mx + logf(expf(ls - mx) + expf(lf - mx));
    wa = expf(ls - lt);
    wf = expf(lf - lt);
  }
  P8<T> fv, out;
  fv.raw = __builtin_nontemporal_load(
      reinterpret_cast<const u32x4*>(of + b * a.f_sb + t * a.f_st + h * a.f_sh + dg * 8));
#pragma unroll
  for (int e = 0; e < 8; ++e)
    out.e[e] = static_cast<T>(fmaf(static_cast<float>(fv.e[e]), wf, static_cast<float>(s.e[e]) * wa));
  *reinterpret_cast<u32x4*>(ot + off) = out.raw;
}

template <typename T>
hipError_t launch_typed(const MergeArgs& a, hipStream_t stream) {
  const int64_t total = (int64_t)a.B * a.T * a.H * (a.D / 8);
  if (total == 0) return hipSuccess;
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL((lse_merge_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_lse_merge(const MergeArgs& a, Elem dtype, hipStream_t stream) {
  return dtype == Elem::BF16 ? launch_typed<__bf16>(a, stream) : launch_typed<_Float16>(a, stream);
}

}  // namespace ttcd
