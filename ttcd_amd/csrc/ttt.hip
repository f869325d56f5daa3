// ttt.hip - SwiGLU and the TTT MLP's feature pass for gfx950.
//
// swiglu_kernel replaces fla's swiglu_fwd_kernel (fla/modules/activations.py:
// 412-426, called by swiglu / swiglu_linear in every MLP of the model):
//   z = (g * s) * u,  s = 1 / (1 + exp(-g)),  in fp32, rounded to the dtype.
// swiglu reads gate / up once, with non-temporal loads; the feature pass's
// gate / up reads stay cached, since neighbouring runs re-read their halo
// rows. Outputs are stored normally: the next op reads them soon, from the
// last-level cache when they fit.
//
// ttt_features_kernel does, in one pass, what the TTT MLP's forward does in
// five launches before its update GEMMs (custom_models/ipttcd/
// modeling_ipttcdv9_lowcopy_scanfuse.py:48-70 with the chunk-local conv of
// profiling/fused_conv.py as patched in by profiling/patches.py:411-432, and
// the group loop's diff at :117-120):
//   z      = swiglu(gate_t, up_t)                teacher features (rounded)
//   zr     = swiglu(gate_s, up_s)                student features (rounded)
//   z_tgt  = conv_t(z), z_hat = conv_s(zr)       chunk-local causal depthwise
//                                                conv, fp32 taps j = 0..K-1,
//                                                each rounded to the dtype
//   diff   = z_tgt - z_hat                       fp32 of the rounded values,
//                                                rounded (chunks 0..T-2 only:
//                                                the last chunk never updates)
// It writes z (the output path reads it), z_hat (the update GEMM reads it)
// and diff; z_tgt and zr never reach HBM. Every intermediate is rounded where
// the reference stores it, so each output equals the reference's chain of
// launches bit for bit (given the same exp).
//
// Layout: rows are tokens, b-major, then chunk, then position in chunk;
// gate / up are the two halves of one (rows, 2*I) GEMM output (row stride
// `gu_stride` elements, gate at column 0, up at column I). Each thread owns
// 8 channels (16 bytes) of a run of kRows consecutive positions of one chunk
// and keeps the K-1 previous rows of both feature streams in registers, as
// the standalone conv kernel does. The halo rows at the start of a run are
// recomputed from gate / up (L2 hits: the neighbouring run streams them).
//
// The update scan of the group loop (scanfuse.py:121-172) around its GEMMs:
// ttt_pd_beta_t_kernel writes pd * beta (the projected difference scaled by
// the per-token learning rate, :126-127, one bf16 multiply) transposed per
// chunk, (chunk, H, C), so the update GEMM dW_c = pd_c^T z_hat_c (:146-149)
// runs as one batched GEMM on contiguous operands; ttt_scan_kernel then does
// what the reference does in three torch launches per group plus one add per
// chunk (:157-170): the running sum over the group's chunk updates with the
// sum stored in the dtype after every step (torch's GPU scan of a bf16
// tensor), cs_j = lr * sum_j rounded, W_step = W_cur + cs rounded, and the
// next group's W_cur; it writes every chunk's W_step transposed, (step, I, H),
// so the per-chunk output GEMMs z_c W_step^T (:161-165) are one batched GEMM
// on contiguous operands as well. Both transpose through 64 x 64 LDS tiles.
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

// Rounded to T as a separate step from the fp32 result (no fused
// multiply-and-convert), as the reference stores an fp32 value.
template <typename T>
__device__ __forceinline__ T round_to(float v) {
  asm volatile("" : "+v"(v));
  return static_cast<T>(v);
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  const float s = 1.0f / (1.0f + expf(-g));
  return (g * s) * u;
}

constexpr int kRows = 16;  // positions per thread

template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const T* __restrict__ gate,
                                                     const T* __restrict__ up,
                                                     T* __restrict__ out, int64_t rows, int cols,
                                                     int64_t g_st, int64_t u_st, int64_t o_st) {
  const int ng = cols / 8;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= rows * ng) return;
  const int64_t r = gid / ng;
  const int c = (int)(gid % ng) * 8;
  V8<T> g, u, o;
  g.raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gate + r * g_st + c));
  u.raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(up + r * u_st + c));
#pragma unroll
  for (int e = 0; e < 8; ++e)
    o.e[e] = round_to<T>(silu_mul(static_cast<float>(g.e[e]), static_cast<float>(u.e[e])));
  *reinterpret_cast<u32x4*>(out + r * o_st + c) = o.raw;
}

// One fused feature row: the rounded swiglu of a (gate, up) row slice.
template <typename T>
__device__ __forceinline__ void swiglu_row(const T* gu, int I, float (&f)[8], V8<T>& rounded) {
  V8<T> g, u;
  g.raw = *reinterpret_cast<const u32x4*>(gu);
  u.raw = *reinterpret_cast<const u32x4*>(gu + I);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    rounded.e[e] = round_to<T>(silu_mul(static_cast<float>(g.e[e]), static_cast<float>(u.e[e])));
    f[e] = static_cast<float>(rounded.e[e]);
  }
}

// CT / CS: the teacher / student conv is present (else identity).
template <typename T, typename W, int K, bool CT, bool CS>
__global__ __launch_bounds__(256) void ttt_features_kernel(
    const T* __restrict__ gu_t, const T* __restrict__ gu_s, int64_t gu_st,
    const W* __restrict__ w_t, const W* __restrict__ w_s, T* __restrict__ z,
    T* __restrict__ z_hat, T* __restrict__ diff, int B, int nchunk, int C, int I, int nseg) {
  const int ng = I / 8;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)B * nchunk * nseg * ng;
  if (gid >= total) return;
  const int dg = (int)(gid % ng);
  int64_t rest = gid / ng;
  const int seg = (int)(rest % nseg);
  rest /= nseg;
  const int ch = (int)(rest % nchunk);
  const int b = (int)(rest / nchunk);
  const int d0 = dg * 8;
  const int c0 = seg * kRows;
  const int64_t row0 = ((int64_t)b * nchunk + ch) * C;  // first token row of the chunk
  const bool has_diff = ch < nchunk - 1;
  const int64_t drow0 = ((int64_t)b * (nchunk - 1) + ch) * C;

  float wt[K][8], ws[K][8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < K; ++j) {
      wt[j][e] = CT ? static_cast<float>(w_t[(int64_t)(d0 + e) * K + j]) : 0.f;
      ws[j][e] = CS ? static_cast<float>(w_s[(int64_t)(d0 + e) * K + j]) : 0.f;
    }

  // wt_win / ws_win[t]: rounded features of position c - (K-1) + t
  float twin[K][8], swin[K][8];
#pragma unroll
  for (int t = 0; t < K - 1; ++t) {
    const int c = c0 - (K - 1) + t;
    if (c >= 0) {
      V8<T> dummy;
      swiglu_row(gu_t + (row0 + c) * gu_st + d0, I, twin[t], dummy);
      swiglu_row(gu_s + (row0 + c) * gu_st + d0, I, swin[t], dummy);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) twin[t][e] = swin[t][e] = 0.f;
    }
  }

  const int rows = min(kRows, C - c0);
  for (int r = 0; r < rows; ++r) {
    const int64_t row = row0 + c0 + r;
    V8<T> zt, zs;
    swiglu_row(gu_t + row * gu_st + d0, I, twin[K - 1], zt);
    swiglu_row(gu_s + row * gu_st + d0, I, swin[K - 1], zs);
    *reinterpret_cast<u32x4*>(z + row * I + d0) = zt.raw;
    V8<T> tg, sh, df;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float at = 0.f, as = 0.f;
      if (CT) {
#pragma unroll
        for (int j = 0; j < K; ++j) at = fmaf(twin[j][e], wt[j][e], at);
        tg.e[e] = round_to<T>(at);
      } else {
        tg.e[e] = zt.e[e];
      }
      if (CS) {
#pragma unroll
        for (int j = 0; j < K; ++j) as = fmaf(swin[j][e], ws[j][e], as);
        sh.e[e] = round_to<T>(as);
      } else {
        sh.e[e] = zs.e[e];
      }
      df.e[e] = round_to<T>(static_cast<float>(tg.e[e]) - static_cast<float>(sh.e[e]));
    }
    *reinterpret_cast<u32x4*>(z_hat + row * I + d0) = sh.raw;
    if (has_diff)
      *reinterpret_cast<u32x4*>(diff + (drow0 + c0 + r) * I + d0) = df.raw;
#pragma unroll
    for (int t = 0; t < K - 1; ++t)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        twin[t][e] = twin[t + 1][e];
        swin[t][e] = swin[t + 1][e];
      }
  }
}

template <typename T, typename W, int K, bool CT, bool CS>
hipError_t launch_feat(const TttFeatureArgs& a, hipStream_t st) {
  const int nseg = (a.C + kRows - 1) / kRows;
  const int64_t total = (int64_t)a.B * a.nchunk * nseg * (a.I / 8);
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL((ttt_features_kernel<T, W, K, CT, CS>), dim3((unsigned)blocks), dim3(256), 0,
                     st, static_cast<const T*>(a.gu_t), static_cast<const T*>(a.gu_s), a.gu_st,
                     static_cast<const W*>(a.w_t), static_cast<const W*>(a.w_s),
                     static_cast<T*>(a.z), static_cast<T*>(a.z_hat), static_cast<T*>(a.diff), a.B,
                     a.nchunk, a.C, a.I, nseg);
  return hipGetLastError();
}

template <typename T, typename W, int K>
hipError_t launch_ck(const TttFeatureArgs& a, hipStream_t st) {
  const bool ct = a.w_t != nullptr, cs = a.w_s != nullptr;
  if (ct && cs) return launch_feat<T, W, K, true, true>(a, st);
  if (ct) return launch_feat<T, W, K, true, false>(a, st);
  if (cs) return launch_feat<T, W, K, false, true>(a, st);
  return launch_feat<T, W, 1, false, false>(a, st);
}

template <typename T, typename W>
hipError_t launch_k(const TttFeatureArgs& a, hipStream_t st) {
  switch (a.K) {
    case 1: return launch_ck<T, W, 1>(a, st);
    case 2: return launch_ck<T, W, 2>(a, st);
    case 3: return launch_ck<T, W, 3>(a, st);
    case 4: return launch_ck<T, W, 4>(a, st);
    case 5: return launch_ck<T, W, 5>(a, st);
    case 6: return launch_ck<T, W, 6>(a, st);
    case 7: return launch_ck<T, W, 7>(a, st);
    default: return launch_ck<T, W, 8>(a, st);
  }
}

template <typename T>
hipError_t launch_wt(const TttFeatureArgs& a, Elem wt, hipStream_t st) {
  switch (wt) {
    case Elem::BF16: return launch_k<T, __bf16>(a, st);
    case Elem::F16: return launch_k<T, _Float16>(a, st);
    default: return launch_k<T, float>(a, st);
  }
}

template <typename T>
hipError_t launch_sw(const void* g, const void* u, void* o, int64_t rows, int cols, int64_t g_st,
                     int64_t u_st, int64_t o_st, hipStream_t st) {
  const int64_t total = rows * (cols / 8);
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL(swiglu_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, st,
                     static_cast<const T*>(g), static_cast<const T*>(u), static_cast<T*>(o), rows,
                     cols, g_st, u_st, o_st);
  return hipGetLastError();
}

// 64 x 64 tile transposes for the update scan. Thread (tx, ty) = (tid % 64,
// tid / 64) handles rows ty, ty + 4, ... of a tile; the LDS tile is fp32 with
// a 65-word row pitch, so the transposed reads are free of bank conflicts.
constexpr int kTile = 64;

template <typename T>
__global__ __launch_bounds__(256) void ttt_pd_beta_t_kernel(TttProjBetaArgs a) {
  __shared__ float tile[kTile][kTile + 1];
  const int tx = threadIdx.x % kTile, ty = threadIdx.x / kTile;
  const int h0 = blockIdx.x * kTile, t0 = blockIdx.y * kTile, bk = blockIdx.z;
  const int b = bk / a.nupd, c = bk % a.nupd;
  const T* pd = static_cast<const T*>(a.pd) + (int64_t)bk * a.C * a.pd_stride;
  const T* beta = a.beta ? static_cast<const T*>(a.beta) + b * a.beta_sb + (int64_t)c * a.C
                         : nullptr;
#pragma unroll
  for (int r = 0; r < kTile / 4; ++r) {
    const int t = t0 + ty + 4 * r, h = h0 + tx;
    float v = 0.f;
    if (t < a.C && h < a.H) {
      v = static_cast<float>(pd[(int64_t)t * a.pd_stride + h]);
      // bf16 * bf16 is exact in fp32: one rounding, as the reference's multiply
      if (beta) v = static_cast<float>(round_to<T>(v * static_cast<float>(beta[t])));
    }
    tile[ty + 4 * r][tx] = v;
  }
  __syncthreads();
  T* out = static_cast<T*>(a.pdt) + (int64_t)bk * a.H * a.C;
#pragma unroll
  for (int r = 0; r < kTile / 4; ++r) {
    const int h = h0 + ty + 4 * r, t = t0 + tx;
    if (h < a.H && t < a.C) out[(int64_t)h * a.C + t] = static_cast<T>(tile[tx][ty + 4 * r]);
  }
}

template <typename T>
__device__ __forceinline__ void store_tile_t(float (&tile)[kTile][kTile + 1], const float (&v)[16],
                                             T* out, int h0, int i0, int H, int I, int tx,
                                             int ty) {
  // v[r] is element (h0 + ty + 4r, i0 + tx); out is (I, H): row i, column h
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 16; ++r) tile[ty + 4 * r][tx] = v[r];
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = i0 + ty + 4 * r, h = h0 + tx;
    if (i < I && h < H) out[(int64_t)i * H + h] = static_cast<T>(tile[tx][ty + 4 * r]);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void ttt_scan_kernel(TttScanArgs a) {
  __shared__ float tile[kTile][kTile + 1];
  const int tx = threadIdx.x % kTile, ty = threadIdx.x / kTile;
  const int i0 = blockIdx.x * kTile, h0 = blockIdx.y * kTile;
  const int i = i0 + tx;
  const T* wc = static_cast<const T*>(a.w_cur);
  const T* dw = static_cast<const T*>(a.dw);
  T* steps = static_cast<T*>(a.steps_t);
  const int64_t HI = (int64_t)a.H * a.I;
  float w[16], acc[16], ws[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int h = h0 + ty + 4 * r;
    w[r] = (h < a.H && i < a.I) ? static_cast<float>(wc[(int64_t)h * a.I + i]) : 0.f;
    acc[r] = 0.f;
    ws[r] = w[r];
  }
  store_tile_t<T>(tile, w, steps, h0, i0, a.H, a.I, tx, ty);  // step 0: W_cur
  for (int j = 0; j < a.nupd; ++j) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int h = h0 + ty + 4 * r;
      const float d = (h < a.H && i < a.I) ? static_cast<float>(dw[j * HI + (int64_t)h * a.I + i])
                                           : 0.f;
      acc[r] = static_cast<float>(round_to<T>(acc[r] + d));          // running sum, stored
      const float cs = static_cast<float>(round_to<T>(a.lr * acc[r]));  // lr * cumsum
      ws[r] = static_cast<float>(round_to<T>(w[r] + cs));            // W_cur + cs_j
    }
    if (j + 1 < a.nsteps)
      store_tile_t<T>(tile, ws, steps + (int64_t)(j + 1) * HI, h0, i0, a.H, a.I, tx, ty);
  }
  if (a.w_next != nullptr) {
    T* wn = static_cast<T*>(a.w_next);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int h = h0 + ty + 4 * r;
      if (h < a.H && i < a.I) wn[(int64_t)h * a.I + i] = static_cast<T>(ws[r]);
    }
  }
}

template <typename T>
hipError_t launch_pdbt(const TttProjBetaArgs& a, hipStream_t st) {
  const dim3 grid((a.H + kTile - 1) / kTile, (a.C + kTile - 1) / kTile, a.B * a.nupd);
  hipLaunchKernelGGL(ttt_pd_beta_t_kernel<T>, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_scan(const TttScanArgs& a, hipStream_t st) {
  const dim3 grid((a.I + kTile - 1) / kTile, (a.H + kTile - 1) / kTile, 1);
  hipLaunchKernelGGL(ttt_scan_kernel<T>, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_swiglu(const void* gate, const void* up, void* out, int64_t rows, int cols,
                         int64_t gate_stride, int64_t up_stride, int64_t out_stride, Elem dtype,
                         hipStream_t stream) {
  return dtype == Elem::BF16
             ? launch_sw<__bf16>(gate, up, out, rows, cols, gate_stride, up_stride, out_stride,
                                 stream)
             : launch_sw<_Float16>(gate, up, out, rows, cols, gate_stride, up_stride, out_stride,
                                   stream);
}

hipError_t launch_ttt_features(const TttFeatureArgs& a, Elem dtype, Elem w_dtype,
                               hipStream_t stream) {
  return dtype == Elem::BF16 ? launch_wt<__bf16>(a, w_dtype, stream)
                             : launch_wt<_Float16>(a, w_dtype, stream);
}

hipError_t launch_ttt_proj_beta_t(const TttProjBetaArgs& a, Elem dtype, hipStream_t stream) {
  return dtype == Elem::BF16 ? launch_pdbt<__bf16>(a, stream) : launch_pdbt<_Float16>(a, stream);
}

hipError_t launch_ttt_scan(const TttScanArgs& a, Elem dtype, hipStream_t stream) {
  return dtype == Elem::BF16 ? launch_scan<__bf16>(a, stream) : launch_scan<_Float16>(a, stream);
}

}  // namespace ttcd
