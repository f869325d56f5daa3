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

#ifndef TTCD_WAVES_PER_EU
#define TTCD_WAVES_PER_EU 2
#endif
#ifndef TTCD_INTERLEAVE_PV
#define TTCD_INTERLEAVE_PV 1
#endif

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
  static constexpr int CPR = D / 8;          // 16-byte chunks per K row
  static constexpr int VSTR = kBlockN + 8;   // V^T tile row stride (elements)
  static constexpr int K_ELEMS = kBlockN * D;  // K tile, rows unpadded, chunks XOR-swizzled
  static constexpr int V_ELEMS = D * VSTR;
  static constexpr int STAGE = K_ELEMS + V_ELEMS;
  static constexpr int DK = D / 16;  // MFMA k-steps of S^T = K Q^T
  static constexpr int DT = D / 32;  // 32-row d tiles of O^T
  static constexpr int NTH = kWaves * 64;
  static constexpr int KDMA = kBlockN * CPR / NTH;          // direct K loads per thread
  static constexpr int VU = (kBlockN / 2) * CPR / NTH;      // (2 keys x 8 d) V units per thread
  static_assert(KDMA * NTH == kBlockN * CPR, "K tile must split evenly");
  static_assert(VU * NTH == (kBlockN / 2) * CPR, "V tile must split evenly");
};

template <int D>
struct VStage {
  u32x4 va[Geo<D>::VU];
  u32x4 vb[Geo<D>::VU];
};

// Position of key kk (0..63 inside the tile) in a V^T row: bits 2 and 3
// swapped, matching the key held by MFMA k-slot (lane/32)*8 + e of the P^T
// operand built from the S^T accumulator registers.
__device__ __forceinline__ int vt_pos(int kk) {
  return (kk & ~15) | (kk & 3) | ((kk >> 3) & 1) << 2 | ((kk >> 2) & 1) << 3;
}

// Per-thread byte offsets of this thread's tile loads relative to the tile's
// first key row; computed once, so a tile costs one scalar base update.
template <int D>
struct LoadPlan {
  uint32_t k_off[Geo<D>::KDMA];  // K chunk this lane moves per direct load
  int k_row[Geo<D>::KDMA];
  uint32_t v_off[Geo<D>::VU];    // V row 2*(u&31), chunk u>>5
  int v_row[Geo<D>::VU];
};

template <int D>
__device__ __forceinline__ LoadPlan<D> make_load_plan(int64_t k_st, int64_t v_st, int wave,
                                                      int lane, int tid) {
  using G = Geo<D>;
  LoadPlan<D> p;
#pragma unroll
  for (int i = 0; i < G::KDMA; ++i) {
    const int slot = (i * kWaves + wave) * 64 + lane;
    const int row = slot / G::CPR;
    const int chunk = (slot % G::CPR) ^ (row % G::CPR);
    p.k_row[i] = row;
    p.k_off[i] = (uint32_t)(row * k_st * 2 + chunk * 16);
  }
#pragma unroll
  for (int i = 0; i < G::VU; ++i) {
    const int u = tid + i * G::NTH;
    p.v_row[i] = 2 * (u & 31);
    p.v_off[i] = (uint32_t)(p.v_row[i] * v_st * 2 + (u >> 5) * 16);
  }
  return p;
}

// K tile: global -> LDS without registers (global_load_lds_dwordx4). Each wave
// instruction writes 64 consecutive 16-byte LDS slots; slot s of row r holds
// global chunk s ^ (r mod CPR), which makes the 16 lanes of an MFMA operand
// read (16 rows, one chunk) hit 16 distinct bank groups. In edge tiles, rows
// outside [0, T) are clamped to a valid row; every score they produce is masked.
template <int D, typename T>
__device__ __forceinline__ void issue_k_tile(T* ks, const T* kp, int64_t k_st, int j0, int T_,
                                             int wave, const LoadPlan<D>& lp, bool interior) {
  using G = Geo<D>;
  const char* tile = reinterpret_cast<const char*>(kp + (int64_t)j0 * k_st);
#pragma unroll
  for (int i = 0; i < G::KDMA; ++i) {
    const char* src;
    if (interior) {
      src = tile + lp.k_off[i];
    } else {
      int j = j0 + lp.k_row[i];
      j = j < 0 ? 0 : (j >= T_ ? T_ - 1 : j);
      src = tile + lp.k_off[i] + (int64_t)(j - j0 - lp.k_row[i]) * k_st * 2;
    }
    const int base = (i * kWaves + wave) * 64;  // first chunk slot of this instruction
    __builtin_amdgcn_global_load_lds(
        (const __attribute__((address_space(1))) void*)src,
        (__attribute__((address_space(3))) void*)(ks + base * 8), 16, 0, 0);
  }
}

template <int D, typename T>
__device__ __forceinline__ void load_v_tile(VStage<D>& r, const T* vp, int64_t v_st, int j0,
                                            int T_, const LoadPlan<D>& lp, bool interior) {
  using G = Geo<D>;
  const char* tile = reinterpret_cast<const char*>(vp + (int64_t)j0 * v_st);
#pragma unroll
  for (int i = 0; i < G::VU; ++i) {
    if (interior) {
      r.va[i] = *reinterpret_cast<const u32x4*>(tile + lp.v_off[i]);
      r.vb[i] = *reinterpret_cast<const u32x4*>(tile + lp.v_off[i] + v_st * 2);
    } else {
      // unconditional loads from clamped rows, zeroed outside [0, T): no branches
      const int ja = j0 + lp.v_row[i];
      const int jca = ja < 0 ? 0 : (ja >= T_ ? T_ - 1 : ja);
      const int jcb = ja + 1 < 0 ? 0 : (ja + 1 >= T_ ? T_ - 1 : ja + 1);
      const char* row0 = tile + lp.v_off[i] - (int64_t)lp.v_row[i] * v_st * 2;
      const u32x4 a = *reinterpret_cast<const u32x4*>(row0 + (int64_t)(jca - j0) * v_st * 2);
      const u32x4 b = *reinterpret_cast<const u32x4*>(row0 + (int64_t)(jcb - j0) * v_st * 2);
      const u32x4 z = {0u, 0u, 0u, 0u};
      r.va[i] = (ja >= 0 && ja < T_) ? a : z;
      r.vb[i] = (ja + 1 >= 0 && ja + 1 < T_) ? b : z;
    }
  }
}

// V tile registers -> LDS transposed (V^T rows = d, key positions vt_pos).
template <int D, typename T>
__device__ __forceinline__ void store_v_tile(const VStage<D>& r, T* vt, int tid) {
  using G = Geo<D>;
#pragma unroll
  for (int i = 0; i < G::VU; ++i) {
    const int u = tid + i * G::NTH;
    const int kk = 2 * (u & 31);
    const int dch = u >> 5;
    T* base = vt + (dch * 8) * G::VSTR + vt_pos(kk);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t a = r.va[i][e], b = r.vb[i][e];
      // v_perm_b32 byte selects over {b:a}: low halves (d = 8*dch + 2e), high halves (+1)
      const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x05040100u);
      const uint32_t hi = __builtin_amdgcn_perm(b, a, 0x07060302u);
      *reinterpret_cast<uint32_t*>(base + (2 * e) * G::VSTR) = lo;
      *reinterpret_cast<uint32_t*>(base + (2 * e + 1) * G::VSTR) = hi;
    }
  }
}

// Scheduling masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

// Interleave N LDS operand reads with the N MFMAs that consume them, two
// reads in flight: r r (M r)* M M.
template <int N>
__device__ __forceinline__ void pipeline_reads_with_mfma() {
  __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
#pragma unroll
  for (int i = 0; i < N - 2; ++i) {
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
}

// S^T (64 keys x 32 queries) of the current tile: two 32x32 fp32 tiles.
template <int D, typename T>
__device__ __forceinline__ void compute_scores(f32x16 (&s)[2], const T* ks,
                                               const typename VecT<T>::v8 (&qf)[Geo<D>::DK],
                                               int lane) {
  using G = Geo<D>;
  using v8 = typename VecT<T>::v8;
  constexpr int N = 2 * G::DK;
  const int r = lane & 31;
  // Chunk 2*ks + half of row r lives in slot (2*ks) ^ y, y = half ^ (r mod CPR).
  // Row bases are multiples of the row size, so the byte offset of every
  // (kt, ks) operand is one XOR of a per-lane base with a constant (plus the
  // kt row block). The empty asm keeps the compiler from hoisting all DK
  // XOR results out of the tile loop into DK live registers.
  uint32_t xbase = (uint32_t)(r * D * 2) | (uint32_t)(((lane >> 5) ^ (r % G::CPR)) << 4);
  asm volatile("" : "+v"(xbase));
  const char* kb = reinterpret_cast<const char*>(ks);
  v8 a[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint32_t off = (xbase ^ (uint32_t)((i % G::DK) << 5)) + (i / G::DK) * 32 * D * 2;
    a[i] = *reinterpret_cast<const v8*>(kb + off);
  }
  s[0] = f32x16{};
  s[1] = f32x16{};
#pragma unroll
  for (int i = 0; i < N; ++i) s[i / G::DK] = mfma32(a[i], qf[i % G::DK], s[i / G::DK]);
  pipeline_reads_with_mfma<N>();
}

// Lazy online-softmax rescale: the running max used for exp2 is only moved
// when some row's true max exceeds it by more than 2^kRescaleLog2 (so p stays
// <= 256 and l, O^T cannot overflow). Softmax is invariant to the reference
// max, so results are the same up to rounding, and the O^T rescale (a VALU
// pass over the whole accumulator) leaves the common path: with the
// diagonal tile first, rows almost never raise their max by 2^8 later.
constexpr float kRescaleLog2 = 8.0f;

// One online-softmax step of band {lo, hi} over the tile starting at key j0:
// masks S in place (if the tile is not entirely inside the band), updates the
// running max m / per-lane partial sum l, rescales O^T when needed and
// accumulates P^T through V^T.
template <int D, typename T>
__device__ __forceinline__ void softmax_pv(f32x16 (&s)[2], f32x16 (&o)[Geo<D>::DT], float& m,
                                           float& l, float c, const T* vt, int lane,
                                           bool need_mask, int qrow, int j0, int T_, Band band) {
  using G = Geo<D>;
  using v8 = typename VecT<T>::v8;
  const int half = lane >> 5;
  // need_mask is wave-uniform; readfirstlane makes that visible to the compiler so
  // this stays a scalar branch instead of being if-converted onto every tile.
  if (__builtin_expect(__builtin_amdgcn_readfirstlane((int)need_mask), 0)) {
    const int jb = j0 + 4 * half;
    const unsigned width = (unsigned)(band.hi - band.lo);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int j = jb + kt * 32 + 8 * (i >> 2) + (i & 3);
        const bool ok = (unsigned)(qrow - j - band.lo) < width && (unsigned)j < (unsigned)T_;
        s[kt][i] = ok ? s[kt][i] : -INFINITY;
      }
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kt][i]);
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float m_new = fmaxf(m, mx);
  // m = -inf and a finite m_new give +inf (rescale); both -inf give NaN (no rescale)
  const bool grow = (m_new - m) * c > kRescaleLog2;
  if (__builtin_expect(__any(grow), 0)) {
    const float mc_new = (m_new == -INFINITY) ? 0.f : m_new * c;
    const float alpha = fast_exp2(fmaf(m, c, -mc_new));
    l *= alpha;
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt) o[dt] *= alpha;
    m = m_new;
  }
  const float mc = (m == -INFINITY) ? 0.f : m * c;
  float psum = 0.f;
  const T* base = vt + (lane & 31) * G::VSTR + half * 8;
#if TTCD_INTERLEAVE_PV
  // Softmax and PV interleaved per 16-key MFMA step: only one P^T fragment and
  // one step's V^T fragments are live, and the exp2 of step ks+1 can overlap
  // the MFMAs of step ks.
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    v8 pf;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = fast_exp2(fmaf(s[ks >> 1][(ks & 1) * 8 + e], c, -mc));
      psum += p;
      pf[e] = static_cast<T>(p);
    }
    v8 b[G::DT];
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt)
      b[dt] = *reinterpret_cast<const v8*>(base + dt * 32 * G::VSTR + ks * 16);
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt) o[dt] = mfma32(b[dt], pf, o[dt]);
  }
#else
  v8 pf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = fast_exp2(fmaf(s[ks >> 1][(ks & 1) * 8 + e], c, -mc));
      psum += p;
      pf[ks][e] = static_cast<T>(p);
    }
  }
  constexpr int N = 4 * G::DT;
  v8 b[N];
#pragma unroll
  for (int i = 0; i < N; ++i)
    b[i] = *reinterpret_cast<const v8*>(base + (i >> 2) * 32 * G::VSTR + (i & 3) * 16);
#pragma unroll
  for (int i = 0; i < N; ++i) o[i >> 2] = mfma32(b[i], pf[i & 3], o[i >> 2]);
  pipeline_reads_with_mfma<N>();
#endif
  l += psum;
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

template <int D, typename T, bool DUAL>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256),
                          amdgpu_waves_per_eu(TTCD_WAVES_PER_EU, TTCD_WAVES_PER_EU)))
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

  const LoadPlan<D> lp = make_load_plan<D>(a.k_st, a.v_st, wave, lane, tid);
  VStage<D> vr;
  if (n_hi >= n_lo) {
    const int j0 = sc.tile_start(n_hi);
    const bool interior = j0 >= 0 && j0 + kBlockN <= T_;
    issue_k_tile<D, T>(smem, kp, a.k_st, j0, T_, wave, lp, interior);
    load_v_tile<D, T>(vr, vp, a.v_st, j0, T_, lp, interior);
    store_v_tile<D, T>(vr, smem + G::K_ELEMS, tid);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  for (int n = n_hi, it = 0; n >= n_lo; --n, ++it) {
    T* ks = smem + (it & 1) * G::STAGE;
    T* vt = ks + G::K_ELEMS;
    T* nks = smem + ((it + 1) & 1) * G::STAGE;
    const bool has_next = n - 1 >= n_lo;
    if (has_next) {
      const int jn = sc.tile_start(n - 1);
      const bool interior = jn >= 0 && jn + kBlockN <= T_;
      issue_k_tile<D, T>(nks, kp, a.k_st, jn, T_, wave, lp, interior);
      load_v_tile<D, T>(vr, vp, a.v_st, jn, T_, lp, interior);
    }

    const int j0 = sc.tile_start(n);
    if (wave_valid) {
      const bool in1 = wave_touches(r0, sc.p1, j0);
      const bool in2 = DUAL && wave_touches(r0, sc.p2, j0);
      // At most two passes over the tile: phase 1 then (dual kernel, mixed
      // tile only) phase 2, which recomputes S rather than keeping a copy.
      int phase = in1 ? 1 : (in2 ? 2 : 0);
      while (phase != 0) {
        const Band band = phase == 1 ? sc.p1 : sc.p2;
        f32x16 s[2];
        compute_scores<D, T>(s, ks, qf, lane);
        softmax_pv<D, T>(s, o, m, l, a.c, vt, lane, !wave_full(r0, band, j0), qrow, j0, T_,
                         band);
        if (DUAL && phase == 1 && wave_last(r0, sc.p1, j0)) {
          emit<D, T>(o, m, l, a.c, os, a.o_st, lse_s, qrow, T_, lane);
          emitted_s = true;
        }
        phase = (DUAL && phase == 1 && in2) ? 2 : 0;
      }
    }
    if (has_next) store_v_tile<D, T>(vr, nks + G::K_ELEMS, tid);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
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
