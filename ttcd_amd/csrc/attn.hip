// attn.hip - one-pass dual-window / single-band causal GQA attention for
// gfx950 (MI355X), bf16 or f16 inputs, fp32 online softmax.
//
// Replaces the Triton kernel _fused_dual_swa_fwd
// (profiling/fused_dual_attn.py:44-241) and the flash-attention windowed
// calls of the LSE variant (profiling/lse_dual_attn.py:22-29, :143-149).
//
// Mapping onto CDNA4
//   * One workgroup = 4 wavefronts = 128 query tokens of one query head; the
//     K/V tile (64 keys) is staged once in LDS and read by all 4 waves.
//   * Scores are produced TRANSPOSED, S^T = K Q^T, with
//     v_mfma_f32_32x32x16_{bf16,f16}: in the 32x32 accumulator layout every
//     lane owns one query (column lane%32) and 16 of the 32 keys (rows), the
//     other 16 living in lane^32. Row max / row sum are therefore in-register
//     reductions plus one cross-half exchange, and the online-softmax rescale
//     factor is a per-lane scalar.
//   * O^T = V^T P^T accumulates in 4 (D=128) or 2 (D=64) 32x32 fp32 tiles.
//     P^T is consumed straight from the score registers (bf16/f16-rounded);
//     the MFMA k-slot <-> key assignment this implies (bits 2 and 3 of the
//     key index swapped inside each 16-key step) is absorbed by the LDS
//     layout of V^T, which the staging code writes transposed.
//   * LDS tiles are padded (K rows D+8, V^T rows 64+8 elements) so the
//     16-byte operand reads of 16 consecutive lanes hit distinct banks.
//   * K/V tiles are double-buffered: the global loads of tile n-1 are issued
//     before the MFMA work on tile n and written to LDS after it; one
//     workgroup barrier per tile.
//   * Workgroups are remapped so each XCD (own L2) sweeps a contiguous run of
//     (b, kv-head, q-tile, q-head-in-group), i.e. the GQA heads sharing a K/V
//     head and neighbouring query tiles share that XCD's L2.
//
// Numerics follow the reference kernel (fused_dual_attn.py:1-13, :100-107):
// raw-domain running max, p = exp2(s*c - m*c) with c = sm_scale*log2(e),
// the m == -inf -> 0 guard, P rounded to the input dtype before PV, l summed
// from the unrounded fp32 p, epilogue acc * (1/l) rounded to nearest-even.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "internal.h"
#include "schedule.h"

namespace ttcd {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct VecT;
template <>
struct VecT<__bf16> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
};
template <>
struct VecT<_Float16> {
  typedef f16x8 v8;
  typedef f16x4 v4;
};

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup id -> logical tile id such that XCD x (which receives ids
// g = x, x+8, ...) processes one contiguous range of logical ids.
__device__ __forceinline__ int xcd_remap(int g, int total) {
  constexpr int kXcd = 8;
  const int q = total / kXcd, r = total % kXcd;
  const int x = g % kXcd, loc = g / kXcd;
  return x < r ? x * (q + 1) + loc : r * (q + 1) + (x - r) * q + loc;
}

template <int D>
struct Geo {
  static constexpr int KSTR = D + 8;        // K tile row stride (elements)
  static constexpr int VSTR = kBlockN + 8;  // V^T tile row stride (elements)
  static constexpr int K_ELEMS = kBlockN * KSTR;
  static constexpr int V_ELEMS = D * VSTR;
  static constexpr int STAGE = K_ELEMS + V_ELEMS;
  static constexpr int DK = D / 16;  // MFMA k-steps of S^T = K Q^T
  static constexpr int DT = D / 32;  // 32-row d tiles of O^T
  static constexpr int NTH = kWaves * 64;
  static constexpr int KCH = kBlockN * (D / 8) / NTH;  // 16-byte K chunks per thread
  static constexpr int VU = (kBlockN / 2) * (D / 8) / NTH;  // (2 keys x 8 d) V units per thread
  static_assert(KCH * NTH == kBlockN * (D / 8), "K tile must split evenly");
  static_assert(VU * NTH == (kBlockN / 2) * (D / 8), "V tile must split evenly");
};

template <int D>
struct StageRegs {
  u32x4 k[Geo<D>::KCH];
  u32x4 va[Geo<D>::VU];
  u32x4 vb[Geo<D>::VU];
};

// Position of key kk (0..63 inside the tile) in a V^T row: bits 2 and 3
// swapped, matching the key held by MFMA k-slot (lane/32)*8 + e of the P^T
// operand built from the S^T accumulator registers.
__device__ __forceinline__ int vt_pos(int kk) {
  return (kk & ~15) | (kk & 3) | ((kk >> 3) & 1) << 2 | ((kk >> 2) & 1) << 3;
}

template <int D, typename T>
__device__ __forceinline__ void load_tile(StageRegs<D>& r, const T* kp, const T* vp,
                                          int64_t k_st, int64_t v_st, int j0, int T_,
                                          int tid) {
  using G = Geo<D>;
  constexpr int CPR = D / 8;  // 16-byte chunks per key row
#pragma unroll
  for (int i = 0; i < G::KCH; ++i) {
    const int c = tid + i * G::NTH;
    const int j = j0 + c / CPR;
    const int dch = c % CPR;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (j >= 0 && j < T_) val = *reinterpret_cast<const u32x4*>(kp + (int64_t)j * k_st + dch * 8);
    r.k[i] = val;
  }
#pragma unroll
  for (int i = 0; i < G::VU; ++i) {
    const int u = tid + i * G::NTH;
    const int ja = j0 + 2 * (u & 31);
    const int dch = u >> 5;
    u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
    if (ja >= 0 && ja < T_) a = *reinterpret_cast<const u32x4*>(vp + (int64_t)ja * v_st + dch * 8);
    if (ja + 1 >= 0 && ja + 1 < T_)
      b = *reinterpret_cast<const u32x4*>(vp + (int64_t)(ja + 1) * v_st + dch * 8);
    r.va[i] = a;
    r.vb[i] = b;
  }
}

template <int D, typename T>
__device__ __forceinline__ void store_tile(const StageRegs<D>& r, T* ks, T* vt, int tid) {
  using G = Geo<D>;
  constexpr int CPR = D / 8;
#pragma unroll
  for (int i = 0; i < G::KCH; ++i) {
    const int c = tid + i * G::NTH;
    *reinterpret_cast<u32x4*>(ks + (c / CPR) * G::KSTR + (c % CPR) * 8) = r.k[i];
  }
#pragma unroll
  for (int i = 0; i < G::VU; ++i) {
    const int u = tid + i * G::NTH;
    const int kk = 2 * (u & 31);
    const int dch = u >> 5;
    T* base = vt + (dch * 8) * G::VSTR + vt_pos(kk);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t a = r.va[i][e], b = r.vb[i][e];
      const uint32_t lo = (a & 0xffffu) | (b << 16);          // d = 8*dch + 2e
      const uint32_t hi = (a >> 16) | (b & 0xffff0000u);      // d = 8*dch + 2e + 1
      *reinterpret_cast<uint32_t*>(base + (2 * e) * G::VSTR) = lo;
      *reinterpret_cast<uint32_t*>(base + (2 * e + 1) * G::VSTR) = hi;
    }
  }
}

// S^T (64 keys x 32 queries) of the current tile: two 32x32 fp32 tiles.
template <int D, typename T>
__device__ __forceinline__ void compute_scores(f32x16 (&s)[2], const T* ks,
                                               const typename VecT<T>::v8 (&qf)[Geo<D>::DK],
                                               int lane) {
  using G = Geo<D>;
  using v8 = typename VecT<T>::v8;
  const T* base = ks + (lane & 31) * G::KSTR + (lane >> 5) * 8;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    f32x16 acc = {};
#pragma unroll
    for (int kst = 0; kst < G::DK; ++kst) {
      const v8 a = *reinterpret_cast<const v8*>(base + kt * 32 * G::KSTR + kst * 16);
      acc = mfma32(a, qf[kst], acc);
    }
    s[kt] = acc;
  }
}

// One online-softmax step of band {lo, hi} over the tile starting at key j0:
// masks (if MASK), updates the running max m / per-lane partial sum l,
// rescales O^T and accumulates P^T through V^T.
template <bool MASK, int D, typename T>
__device__ __forceinline__ void softmax_pv(const f32x16 (&s)[2], f32x16 (&o)[Geo<D>::DT],
                                           float& m, float& l, float c, const T* vt,
                                           int lane, int qrow, int j0, int T_, Band band) {
  using G = Geo<D>;
  using v8 = typename VecT<T>::v8;
  const int half = lane >> 5;
  float sv[32];
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float x = s[kt][i];
      if (MASK) {
        const int j = j0 + kt * 32 + 8 * (i >> 2) + 4 * half + (i & 3);
        const int d = qrow - j;
        const bool ok = (unsigned)(d - band.lo) < (unsigned)(band.hi - band.lo) &&
                        (unsigned)j < (unsigned)T_;
        x = ok ? x : -INFINITY;
      }
      sv[kt * 16 + i] = x;
      mx = fmaxf(mx, x);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float m_new = fmaxf(m, mx);
  const float mc = (m_new == -INFINITY) ? 0.f : m_new * c;
  const float alpha = fast_exp2(fmaf(m, c, -mc));
  float psum = 0.f;
  v8 pf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = fast_exp2(fmaf(sv[ks * 8 + e], c, -mc));
      psum += p;
      pf[ks][e] = static_cast<T>(p);
    }
  }
  l = fmaf(l, alpha, psum);
  m = m_new;
#pragma unroll
  for (int dt = 0; dt < G::DT; ++dt) o[dt] *= alpha;
  const T* base = vt + (lane & 31) * G::VSTR + half * 8;
#pragma unroll
  for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const v8 a = *reinterpret_cast<const v8*>(base + dt * 32 * G::VSTR + ks * 16);
      o[dt] = mfma32(a, pf[ks], o[dt]);
    }
  }
}

// Normalise and store one output (and its LSE) from the O^T accumulator.
template <int D, typename T>
__device__ __forceinline__ void emit(const f32x16 (&o)[Geo<D>::DT], float m, float l, float c,
                                     T* out, int64_t o_st, float* lse, int qrow, int T_,
                                     int lane) {
  using v4 = typename VecT<T>::v4;
  const float lt = l + __shfl_xor(l, 32);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (qrow >= T_) return;
  const int half = lane >> 5;
  T* dst = out + (int64_t)qrow * o_st + half * 4;
#pragma unroll
  for (int dt = 0; dt < Geo<D>::DT; ++dt) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      v4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = static_cast<T>(o[dt][4 * g + e] * inv);
      *reinterpret_cast<v4*>(dst + dt * 32 + 8 * g) = w;
    }
  }
  if (lse != nullptr && half == 0) {
    const float mc = (m == -INFINITY) ? 0.f : m * c;
    lse[qrow] = lt > 0.f ? mc * 0.69314718055994531f + logf(lt) : -INFINITY;
  }
}

// D=64 fits two waves per SIMD (<= 256 VGPRs); D=128 holds a 64-register
// O^T accumulator plus 32 registers of Q^T and takes one wave per SIMD with
// the full 512-register file.
template <int D>
struct Occ {
  static constexpr int waves = D == 64 ? 2 : 1;
};

template <int D, typename T, bool DUAL>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256),
                          amdgpu_waves_per_eu(Occ<D>::waves, Occ<D>::waves)))
void attn_fwd_kernel(AttnArgs a) {
  using G = Geo<D>;
  using v8 = typename VecT<T>::v8;
  __shared__ __attribute__((aligned(16))) T smem[2 * G::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Schedule sc = a.sched;
  const int T_ = a.T;

  // logical id order (b, kv head, q tile [heaviest first], head in group)
  int rest = xcd_remap(blockIdx.x, gridDim.x);
  const int g = rest % a.G;
  rest /= a.G;
  const int qb = a.nqb - 1 - rest % a.nqb;
  rest /= a.nqb;
  const int hk = rest % a.Hkv;
  const int b = rest / a.Hkv;
  const int h = hk * a.G + g;

  const int t0 = qb * kBlockM;
  const int t_last = min(t0 + kBlockM, T_) - 1;
  const int r0 = t0 + wave * kWaveRows;
  const int qrow = r0 + (lane & 31);
  const bool wave_valid = r0 < T_;

  const T* qp = static_cast<const T*>(a.q) + b * a.q_sb + h * a.q_sh;
  const T* kp = static_cast<const T*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const T* vp = static_cast<const T*>(a.v) + b * a.v_sb + hk * a.v_sh;
  T* ot = static_cast<T*>(a.o_t) + b * a.o_sb + h * a.o_sh;
  T* os = DUAL ? static_cast<T*>(a.o_s) + b * a.o_sb + h * a.o_sh : nullptr;
  float* lse_t = a.lse_t ? a.lse_t + ((int64_t)b * a.Hq + h) * T_ : nullptr;
  float* lse_s = (DUAL && a.lse_s) ? a.lse_s + ((int64_t)b * a.Hq + h) * T_ : nullptr;

  // Q^T operand fragments: lane holds query qrow, d = 16*ks + 8*(lane/32) + e.
  v8 qf[G::DK];
  {
    const T* src = qp + (int64_t)qrow * a.q_st + (lane >> 5) * 8;
#pragma unroll
    for (int ks = 0; ks < G::DK; ++ks) {
      v8 z = {};
      qf[ks] = qrow < T_ ? *reinterpret_cast<const v8*>(src + ks * 16) : z;
    }
  }

  f32x16 o[G::DT];
#pragma unroll
  for (int dt = 0; dt < G::DT; ++dt) o[dt] = f32x16{};
  float m = -INFINITY, l = 0.f;
  bool emitted_s = false;

  int n_hi = 0, n_lo = 1;
  if (!sc.wg_range(t0, t_last, &n_hi, &n_lo)) {
    n_hi = 0;
    n_lo = 1;
  }

  StageRegs<D> sr;
  if (n_hi >= n_lo) {
    load_tile<D, T>(sr, kp, vp, a.k_st, a.v_st, sc.tile_start(n_hi), T_, tid);
    store_tile<D, T>(sr, smem, smem + G::K_ELEMS, tid);
  }
  __syncthreads();

  for (int n = n_hi, it = 0; n >= n_lo; --n, ++it) {
    T* ks = smem + (it & 1) * G::STAGE;
    T* vt = ks + G::K_ELEMS;
    T* nks = smem + ((it + 1) & 1) * G::STAGE;
    const bool has_next = n - 1 >= n_lo;
    if (has_next) load_tile<D, T>(sr, kp, vp, a.k_st, a.v_st, sc.tile_start(n - 1), T_, tid);

    const int j0 = sc.tile_start(n);
    if (wave_valid) {
      const bool in1 = wave_touches(r0, sc.p1, j0);
      const bool in2 = DUAL && wave_touches(r0, sc.p2, j0);
      if (in1 || in2) {
        f32x16 s[2];
        compute_scores<D, T>(s, ks, qf, lane);
        if (in1) {
          if (wave_full(r0, sc.p1, j0))
            softmax_pv<false, D, T>(s, o, m, l, a.c, vt, lane, qrow, j0, T_, sc.p1);
          else
            softmax_pv<true, D, T>(s, o, m, l, a.c, vt, lane, qrow, j0, T_, sc.p1);
          if (DUAL && wave_last(r0, sc.p1, j0)) {
            emit<D, T>(o, m, l, a.c, os, a.o_st, lse_s, qrow, T_, lane);
            emitted_s = true;
          }
        }
        if (DUAL && in2) {
          if (wave_full(r0, sc.p2, j0))
            softmax_pv<false, D, T>(s, o, m, l, a.c, vt, lane, qrow, j0, T_, sc.p2);
          else
            softmax_pv<true, D, T>(s, o, m, l, a.c, vt, lane, qrow, j0, T_, sc.p2);
        }
      }
    }
    if (has_next) store_tile<D, T>(sr, nks, nks + G::K_ELEMS, tid);
    __syncthreads();
  }

  if (wave_valid) {
    if (DUAL && !emitted_s) emit<D, T>(o, m, l, a.c, os, a.o_st, lse_s, qrow, T_, lane);
    emit<D, T>(o, m, l, a.c, ot, a.o_st, lse_t, qrow, T_, lane);
  }
}

template <int D, typename T, bool DUAL>
hipError_t launch_typed(const AttnArgs& a, hipStream_t stream) {
  const int grid = a.B * a.Hq * a.nqb;
  hipLaunchKernelGGL((attn_fwd_kernel<D, T, DUAL>), dim3(grid), dim3(kWaves * 64), 0, stream, a);
  return hipGetLastError();
}

template <int D, typename T>
hipError_t launch_dual_or_band(const AttnArgs& a, hipStream_t stream) {
  return a.sched.dual ? launch_typed<D, T, true>(a, stream) : launch_typed<D, T, false>(a, stream);
}

}  // namespace

hipError_t launch_attn(const AttnArgs& a, int D, Elem dtype, hipStream_t stream) {
  if (D == 128) {
    return dtype == Elem::BF16 ? launch_dual_or_band<128, __bf16>(a, stream)
                               : launch_dual_or_band<128, _Float16>(a, stream);
  }
  return dtype == Elem::BF16 ? launch_dual_or_band<64, __bf16>(a, stream)
                             : launch_dual_or_band<64, _Float16>(a, stream);
}

}  // namespace ttcd
