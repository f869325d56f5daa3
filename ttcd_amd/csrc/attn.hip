// attn.hip - one-pass dual-window / single-band causal GQA attention for
// gfx950 (MI355X), bf16 or f16 inputs, fp32 online softmax.
//
// Replaces the Triton kernel _fused_dual_swa_fwd
// (profiling/fused_dual_attn.py:44-241) and the flash-attention windowed
// calls of the LSE variant (profiling/lse_dual_attn.py:22-29, :143-149).
//
// Mapping onto CDNA4
//   * One workgroup = 4 wavefronts of 32 query columns each: 32 rows of one
//     query head (128 tokens per workgroup), or, when the GQA group size is
//     even, 16 rows of each of two query heads that share the K/V head (64
//     tokens per workgroup; every MFMA operand is shared, and the workgroup's
//     narrower row span sweeps fewer partly-used tiles: one repeated mixed
//     tile instead of two, no skipped edge tiles). D = 128: two workgroups
//     per CU (64 KiB of LDS each, <= 256 VGPRs); D = 64: three (32 KiB each,
//     <= 168 VGPRs). The two or three wavefronts sharing a SIMD come from
//     different workgroups, so one's barrier and DMA time is filled by
//     another's MFMAs.
//   * K and V tiles (64 keys) go global -> LDS by DMA
//     (global_load_lds_dwordx4, no registers) in a two-stage split ring: slot
//     k reads K(k+1) and V(k), so K(k+2) and V(k+1) are fetched at its start
//     and have the whole slot to land. Rows are stored with their 16-byte
//     chunks XOR-swizzled so every operand read below is free of bank
//     conflicts.
//   * Scores are produced TRANSPOSED, S^T = K Q^T, with
//     v_mfma_f32_32x32x16_{bf16,f16}: each lane owns one query (column
//     lane%32) and 16 of the 32 keys (rows); the other 16 live in lane^32.
//     Row max / row sum are in-register reductions plus one
//     v_permlane32_swap, and the online-softmax rescale factor is a
//     per-lane scalar. Q^T stays in registers for the whole sweep.
//   * O^T = V^T P^T accumulates in D/32 32x32 fp32 tiles. P^T comes straight
//     from the score registers (exp2, then rounded to bf16/f16); V^T operands
//     are read from the row-major V tile with ds_read_b64_tr_b16, which
//     transposes 4x4 blocks of 16-bit elements across lanes. The key order
//     of the P^T k-slots (bits 2 and 3 of the key index swapped inside each
//     16-key step) is matched by the rows each transposed read selects.
//   * Software pipeline inside each wavefront: while the MFMAs of the next
//     slot's scores S(k+1) run, the VALU computes exp2 of S(k); the PV MFMAs
//     of slot k then run while the VALU sums the row of S(k) and reduces the
//     row max of S(k+1) (slot_body). In the lazy mode at D = 128 no row max
//     is needed before the exp2, so the PV MFMAs of slot k run under the
//     first half of S(k+1)'s exp2 instead (slot_body_lazy).
//   * Workgroups are remapped so each XCD (own L2) sweeps a contiguous run of
//     (b, kv head, query block, head or head pair in group); heaviest query
//     blocks first.
//   * Packed sequences (cu_seqlens): each workgroup builds its sequence's
//     schedule from the sequence length, with every bound clamped to the
//     packed tensors.
//
// Numerics follow the reference kernel (fused_dual_attn.py:1-13, :100-107):
// raw-domain running max, p = exp2(s*c - m*c) with c = sm_scale*log2(e),
// the m == -inf -> 0 guard, P rounded to the input dtype before PV, l summed
// from the unrounded fp32 p, epilogue acc * (1/l) rounded to nearest-even.
// With rescale_log2 > 0 (lazy rescale, default 8) the reference max m used in
// exp2 may lag a row's running max, with every p <= 2^rescale_log2; softmax
// is invariant to m up to rounding. At D = 64 m moves when the row's max
// grows by more than 2^rescale_log2; at D = 128 when a slot's probabilities
// against m sum above 2^rescale_log2 over a half row (which bounds every p the
// same way without taking the row max in every slot). rescale_log2 = 0 keeps
// the exact running max of the reference.
//
// Built with -fno-honor-nans -mno-amdgpu-ieee (ttcd_amd/build.py): no value
// here is NaN for finite inputs (masked scores are -inf, every test below is
// written without relying on NaN comparisons), and IEEE mode would make each
// fmaxf of an MFMA result re-canonicalise its inputs first.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "internal.h"
#include "schedule.h"

// Software-pipeline depths of the slot body (see slot_body).
#ifndef TTCD_R1
#define TTCD_R1 3  // K operand reads in flight ahead of the score MFMAs
#endif
#ifndef TTCD_R2
#define TTCD_R2 2  // V^T operands in flight ahead of the PV MFMAs
#endif
#ifndef TTCD_P1
#define TTCD_P1 2  // score MFMAs issued before the reference max is settled
#endif

namespace ttcd {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

#define LDS_AS __attribute__((address_space(3)))
#define GLB_AS __attribute__((address_space(1)))

template <typename T>
struct VecT;
template <>
struct VecT<__bf16> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  __device__ static bf16x4 read_tr(const LDS_AS char* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((LDS_AS bf16x4*)p);
  }
};
template <>
struct VecT<_Float16> {
  typedef f16x8 v8;
  typedef f16x4 v4;
  typedef __fp16 h4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
  __device__ static f16x4 read_tr(const LDS_AS char* p) {
    return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((LDS_AS h4*)p));
  }
};

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Values of lanes l and l^32 combined: v_permlane32_swap of v with itself
// leaves the low half's values in one result and the high half's in the other.
__device__ __forceinline__ float xhalf_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ bool xhalf_any(bool v) {
  const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  return (r[0] | r[1]) != 0;
}

// Workgroup id -> logical id such that XCD x (which receives ids g = x, x+8,
// ...) processes one contiguous range of logical ids.
__device__ __forceinline__ int xcd_remap(int g, int total) {
  constexpr int kXcd = 8;
  const int q = total / kXcd, r = total % kXcd;
  const int x = g % kXcd, loc = g / kXcd;
  return x < r ? x * (q + 1) + loc : r * (q + 1) + (x - r) * q + loc;
}

template <int D>
struct Geo {
  static constexpr int RB = D * 2;                 // bytes per K / V row
  static constexpr int CPR = D / 8;                // 16-byte chunks per row
  static constexpr int TILE_B = kBlockN * RB;      // bytes of one K or V tile
  static constexpr int STAGE_B = 2 * TILE_B;       // K tile, then V tile
  static constexpr int NSTAGE = 2;                 // K and V halves refilled one slot ahead
  static constexpr int DK = D / 16;                // MFMA k-steps of S^T = K Q^T
  static constexpr int DT = D / 32;                // 32-row d tiles of O^T
  static constexpr int NTH = kWaves * 64;
  static constexpr int NDMA = kBlockN * CPR / NTH;  // 16-byte DMA loads per lane per tile
  static_assert(NDMA >= 1 && NDMA * NTH == kBlockN * CPR, "tile must split evenly");
};

// LDS chunk swizzles (16-byte chunk c of row r is stored at chunk c ^ swz(r)).
// K: the 16 lanes of one ds_read_b128 pass read 16 consecutive rows at one
// chunk -> 16 distinct bank groups. V: the 32 lanes of one ds_read_b64_tr_b16
// pass read 4 consecutive rows x 4 consecutive chunks -> 16 distinct groups.
template <int D>
__device__ __forceinline__ int swz_k(int r) {
  return D == 128 ? (r & 15) : ((r >> 1) & 7);
}
template <int D>
__device__ __forceinline__ int swz_v(int r) {
  return D == 128 ? ((r & 3) << 2) : (((r >> 1) & 1) << 2);
}

// Per-lane constants: DMA source offsets and LDS operand addresses.
template <int D>
struct Lane {
  uint32_t k_off[Geo<D>::NDMA];  // byte offset of this lane's K chunk in an interior tile
  uint32_t v_off[Geo<D>::NDMA];
  uint32_t xk;                   // K operand address inside a tile (XOR ks << 5 per k-step)
  uint32_t vb[Geo<D>::DT];       // V^T operand address inside a tile per d tile
};

// DMA slot geometry: the lane's i-th load of a tile writes 16-byte LDS slot
// (wave + 8i)*64 + lane, i.e. tile row `row`, physical chunk `pch`.
template <int D>
__device__ __forceinline__ void dma_slot_of(int wave, int lane, int i, int* row, int* pch) {
  const int slot = (wave + kWaves * i) * 64 + lane;
  *row = slot / Geo<D>::CPR;
  *pch = slot % Geo<D>::CPR;
}

template <int D>
__device__ __forceinline__ Lane<D> make_lane(int64_t k_st, int64_t v_st, int wave, int lane) {
  using G = Geo<D>;
  Lane<D> p;
#pragma unroll
  for (int i = 0; i < G::NDMA; ++i) {
    int row, pch;
    dma_slot_of<D>(wave, lane, i, &row, &pch);
    p.k_off[i] = (uint32_t)(row * k_st * 2) + (uint32_t)((pch ^ swz_k<D>(row)) * 16);
    p.v_off[i] = (uint32_t)(row * v_st * 2) + (uint32_t)((pch ^ swz_v<D>(row)) * 16);
  }
  {
    // S^T A operand: lane reads row r = lane%32 (+32 per key block), logical
    // chunk 2*ks + h; physical chunk (2ks + h) ^ s = ((s & ~1) ^ 2ks) | ((h ^ s) & 1).
    const int r = lane & 31, h = lane >> 5, s = swz_k<D>(r);
    p.xk = (uint32_t)(r * G::RB + (((h ^ s) & 1) << 4) + ((s & ~1) << 4));
  }
  {
    // O^T A operand from ds_read_b64_tr_b16: lane i of 16-lane group g names
    // key kb + (i >> 2), d = 32*dt + 16*(g & 1) + 4*(i & 3); lane i then
    // receives keys kb..kb+3 at d = 32*dt + 16*(g & 1) + i.
    const int i = lane & 15, g = lane >> 4;
    const int h = g >> 1, q = i >> 2;
    const int c_lo = 2 * (g & 1) + ((i & 3) >> 1);
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt)
      p.vb[dt] = (uint32_t)((4 * h + q) * G::RB + (((4 * dt + c_lo) ^ swz_v<D>(q)) << 4) +
                            (i & 1) * 8);
  }
  return p;
}

// One 16-byte-per-lane DMA: 64 lanes x 16 bytes from base + voff (per lane)
// into LDS bytes [lds_addr, lds_addr + 1024). Written as inline asm so the
// compiler does not treat every later LDS read as possibly aliasing the DMA
// (which makes it wait for the whole load queue); ordering against LDS reads
// is explicit: s_waitcnt vmcnt + s_barrier in the slot loop.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds_addr) {
  // base and lds_addr are wave-uniform; readfirstlane makes that explicit.
  // (It returns int: widen through uint32_t so the low word is not sign-extended.)
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint64_t bs = (uint64_t)lo | ((uint64_t)hi << 32);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %2"
               :
               : "v"(voff), "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "s"(bs)
               : "memory", "m0");
}
// The N loads of one tile by this lane: chunk off[i] of the tile at `base`
// into LDS bytes lds0 + i * 4096 (i.e. slot (wave + kWaves*i) * 64 + lane of
// a tile whose wave-0 slot 0 is at lds0 - wave * 1024). One asm block, so the
// wait state every M0 write needs before the load that uses it is filled by
// the next LDS address instead of an s_nop.
template <int N>
__device__ __forceinline__ void dma_run(const void* base, const uint32_t (&off)[N],
                                        uint32_t lds0) {
  static_assert(N == 2 || N == 4, "tile loads per lane");
  static_assert(kWaves * 1024 == 0x1000, "LDS stride of a lane's loads");
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint64_t bs = (uint64_t)lo | ((uint64_t)hi << 32);
  const uint32_t l0 = (uint32_t)__builtin_amdgcn_readfirstlane(lds0);
  uint32_t t;
  if constexpr (N == 4) {
    asm volatile(
        "s_mov_b32 m0, %[l]\n\t"
        "s_add_u32 %[t], %[l], 0x1000\n\t"
        "global_load_lds_dwordx4 %[v0], %[b]\n\t"
        "s_mov_b32 m0, %[t]\n\t"
        "s_add_u32 %[t], %[l], 0x2000\n\t"
        "global_load_lds_dwordx4 %[v1], %[b]\n\t"
        "s_mov_b32 m0, %[t]\n\t"
        "s_add_u32 %[t], %[l], 0x3000\n\t"
        "global_load_lds_dwordx4 %[v2], %[b]\n\t"
        "s_mov_b32 m0, %[t]\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %[v3], %[b]"
        : [t] "=&s"(t)
        : [l] "s"(l0), [b] "s"(bs), [v0] "v"(off[0]), [v1] "v"(off[1]), [v2] "v"(off[2]),
          [v3] "v"(off[3])
        : "memory", "m0", "scc");
  } else {
    asm volatile(
        "s_mov_b32 m0, %[l]\n\t"
        "s_add_u32 %[t], %[l], 0x1000\n\t"
        "global_load_lds_dwordx4 %[v0], %[b]\n\t"
        "s_mov_b32 m0, %[t]\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %[v1], %[b]"
        : [t] "=&s"(t)
        : [l] "s"(l0), [b] "s"(bs), [v0] "v"(off[0]), [v1] "v"(off[1])
        : "memory", "m0", "scc");
  }
}
#pragma clang diagnostic pop

// Issue the DMA of one K or V tile (rows j0 .. j0+63) into LDS at byte
// address `dst`. Rows outside [0, T) are clamped to valid rows; every score
// they produce is masked and every probability they meet is exactly 0.
template <int D, typename T, bool IS_K>
__device__ __forceinline__ void dma_tile(uint32_t dst, const T* base, int64_t st, int j0, int T_,
                                         int wave, int lane, const uint32_t (&off)[Geo<D>::NDMA],
                                         bool interior) {
  using G = Geo<D>;
  const T* tile = base + (int64_t)j0 * st;
#pragma unroll
  for (int i = 0; i < G::NDMA; ++i) {
    uint32_t voff = off[i];
    if (!interior) {
      int row, pch;
      dma_slot_of<D>(wave, lane, i, &row, &pch);
      int j = j0 + row;
      j = j < 0 ? 0 : (j >= T_ ? T_ - 1 : j);
      const int sw = IS_K ? swz_k<D>(row) : swz_v<D>(row);
      voff = (uint32_t)((j - j0) * st * 2) + (uint32_t)((pch ^ sw) * 16);
    }
    dma16(tile, voff, dst + (wave + kWaves * i) * 1024);
  }
}

// Key index of S^T accumulator element e of key block kt for this lane.
__device__ __forceinline__ int key_of(int j0, int kt, int e, int half) {
  return j0 + kt * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
}

// Mask S^T of the tile at j0 to band b (in place): key j is visible to row
// qrow iff 0 <= qrow - j - lo < hi - lo and 0 <= j < T. Element (kt, e) of
// this lane holds key j0 + 4*half + o with o = 32kt + 8(e/4) + e%4 a
// compile-time constant, so the band test is one unsigned compare of a
// per-lane value minus o against the uniform width. Keys outside [0, T) can
// only be in a tile that starts before 0 or runs past T - 1 (a uniform
// test); only such tiles take the second pass.
__device__ __forceinline__ void mask_band(f32x16 (&s)[2], int qrow, int j0, int T_, Band b,
                                          int half) {
  const unsigned width = (unsigned)(b.hi - b.lo);
  const unsigned d = (unsigned)qrow - (unsigned)(j0 + 4 * half) - (unsigned)b.lo;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const unsigned o = (unsigned)key_of(0, kt, e, 0);
      s[kt][e] = (d - o) < width ? s[kt][e] : -INFINITY;
    }
  if (j0 < 0 || j0 + kBlockN > T_) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int j = key_of(j0, kt, e, half);
        s[kt][e] = (unsigned)j < (unsigned)T_ ? s[kt][e] : -INFINITY;
      }
  }
}

__device__ __forceinline__ float tile_max(const f32x16 (&s)[2]) {
  float a = -INFINITY, b = -INFINITY;
#pragma unroll
  for (int e = 0; e < 16; e += 2) {
    a = fmaxf(a, fmaxf(s[0][e], s[0][e + 1]));
    b = fmaxf(b, fmaxf(s[1][e], s[1][e + 1]));
  }
  return xhalf_max(fmaxf(a, b));
}

// Normalise and store one output (and its LSE) from the O^T accumulator.
template <int D, typename T>
__device__ __forceinline__ void emit(const f32x16 (&o)[Geo<D>::DT], float m, float l, float c,
                                     T* out, int64_t o_st, float* lse, int qrow, int T_,
                                     int q_off, int lane) {
  using v4 = typename VecT<T>::v4;
  const float lt = xhalf_sum(l);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (qrow >= T_ || qrow < q_off) return;  // rows of this launch only
  const int half = lane >> 5;
  T* dst = out + (int64_t)(qrow - q_off) * o_st + half * 4;
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
    lse[qrow - q_off] = lt > 0.f ? mc * 0.69314718055994531f + logf(lt) : -INFINITY;
  }
}

// Everything the slot body needs besides the per-slot registers.
template <int D, typename T>
struct Ctx {
  using v8 = typename VecT<T>::v8;
  LDS_AS char* lds;
  v8 qf[Geo<D>::DK];  // Q^T B operands: lane holds query qrow, d = 16*ks + 8*(lane/32) + e
  Lane<D> ln;
  float c;
  int qrow, half, T_;
};

// K operand i of the scores (key block i & 1, k-step i >> 1).
template <int D, typename T>
__device__ __forceinline__ typename VecT<T>::v8 read_k(const LDS_AS char* kb, uint32_t xk, int i) {
  using v8 = typename VecT<T>::v8;
  return *(const LDS_AS v8*)(kb + (xk ^ (uint32_t)((i >> 1) << 5)) + (i & 1) * 32 * Geo<D>::RB);
}

// V^T A operand of 16-key step ks from the lane's transposed-read address vb
// of one d tile (two reads: keys +0..3 and +8..11 of the step for this lane).
template <int D, typename T>
__device__ __forceinline__ typename VecT<T>::v8 read_vt(const LDS_AS char* vb, int ks) {
  using G = Geo<D>;
  const auto lo = VecT<T>::read_tr(vb + (16 * ks) * G::RB);
  const auto hi = VecT<T>::read_tr(vb + (16 * ks + 8) * G::RB);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Score element idx (0..31) of the lane in P^T k-step order: k-step idx / 8,
// slot idx % 8 -> accumulator element (k-step & 1) * 8 + slot of key block
// k-step / 2.
__device__ __forceinline__ float score_at(const f32x16 (&s)[2], int idx) {
  return s[(idx >> 3) >> 1][((idx >> 3) & 1) * 8 + (idx & 7)];
}
__device__ __forceinline__ void score_set(f32x16 (&s)[2], int idx, float v) {
  s[(idx >> 3) >> 1][((idx >> 3) & 1) * 8 + (idx & 7)] = v;
}

// One slot of the software pipeline, in issue order (sched_barrier fences
// keep the compiler from regrouping it):
//   phase 1: the scores S(k+1) from the K tile at kb (2*DK MFMAs). After the
//            first two, settle() masks S(k) if needed, settles the reference
//            max of slot k (rescaling O^T when it moves) and returns m*c for
//            its exp2 (+inf for a slot this wave skips); the exp2 / bf16
//            packing of S(k) is then spread over the remaining MFMAs. K
//            operand reads run R1 MFMAs ahead.
//   phase 2: PV(k) from the V tile at vbase (4*DT MFMAs), with the row sum of
//            S(k) and then the row max of S(k+1) spread between them and the
//            V^T operand reads R2 MFMAs ahead.
// Returns this lane's (unmasked) max of S(k+1), not yet combined across halves.
template <int D, typename T, typename Settle>
__device__ __forceinline__ float slot_body(const Ctx<D, T>& x, f32x16 (&sc)[2], f32x16 (&sn)[2],
                                           f32x16 (&o)[Geo<D>::DT], float& l,
                                           const LDS_AS char* kb, const LDS_AS char* vbase,
                                           Settle&& settle) {
  using G = Geo<D>;
  using v8 = typename VecT<T>::v8;
  constexpr int N1 = 2 * G::DK;  // score MFMAs
  constexpr int N2 = 4 * G::DT;  // PV MFMAs
  constexpr int R1 = TTCD_R1;
  constexpr int R2 = TTCD_R2;
  constexpr int P1 = TTCD_P1;          // score MFMAs issued before settle()
  constexpr int H2 = N2 / 2;     // PV MFMAs carrying sums (the rest carry maxima)
  constexpr int A2 = 32 / H2;    // values summed / maxed per PV MFMA

  // The K lane address is opaque per slot, so its eight per-k-step XORs are
  // formed here instead of held in registers (the V^T addresses' per-k-step
  // parts are immediate offsets and need no such fence).
  uint32_t xk = x.ln.xk;
  asm volatile("" : "+v"(xk));
  const LDS_AS char* vb[G::DT];
#pragma unroll
  for (int dt = 0; dt < G::DT; ++dt) vb[dt] = vbase + x.ln.vb[dt];

  // phase 1
  v8 ka[N1];
  v8 pf[4];
  float mc = 0.f;
#pragma unroll
  for (int i = 0; i < R1; ++i) ka[i] = read_k<D, T>(kb, xk, i);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < N1; ++i) {
    const int kt = i & 1, ks = i >> 1;
    sn[kt] = mfma32(ka[i], x.qf[ks], i < 2 ? f32x16{} : sn[kt]);
    if (i + R1 < N1) ka[i + R1] = read_k<D, T>(kb, xk, i + R1);
    if (i == P1 - 1) mc = settle();
    if (i >= P1) {
      // scores (32 * (i - P1) / (N1 - P1)) .. (32 * (i + 1 - P1) / (N1 - P1)) - 1
      const int e0 = 32 * (i - P1) / (N1 - P1), e1 = 32 * (i + 1 - P1) / (N1 - P1);
#pragma unroll
      for (int idx = e0; idx < e1; ++idx) {
        const float p = fast_exp2(fmaf(score_at(sc, idx), x.c, -mc));
        score_set(sc, idx, p);
        if (idx & 1) {
          pf[idx >> 3][(idx & 7) - 1] = static_cast<T>(score_at(sc, idx - 1));
          pf[idx >> 3][idx & 7] = static_cast<T>(p);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // phase 2
  v8 vt[N2];
#pragma unroll
  for (int i = 0; i < R2; ++i) vt[i] = read_vt<D, T>(vb[i % G::DT], i / G::DT);
  float ps0 = 0.f, ps1 = 0.f, mx0 = -INFINITY, mx1 = -INFINITY;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < N2; ++i) {
    const int ks = i / G::DT, dt = i % G::DT;
    o[dt] = mfma32(vt[i], pf[ks], o[dt]);
    if (i < H2) {
#pragma unroll
      for (int j = 0; j < A2; j += 2) {
        const float a0 = score_at(sc, A2 * i + j), a1 = score_at(sc, A2 * i + j + 1);
        ps0 = (i == 0 && j == 0) ? a0 : ps0 + a0;
        ps1 = (i == 0 && j == 0) ? a1 : ps1 + a1;
      }
      // pin the partial sums here: otherwise the chain is sunk to its use
      // after the last MFMA, out of the MFMA shadow
      asm volatile("" : "+v"(ps0), "+v"(ps1));
    } else {
#pragma unroll
      for (int j = 0; j < A2; j += 4) {
        const int idx = A2 * (i - H2) + j;
        mx0 = __builtin_fmaxf(__builtin_fmaxf(mx0, score_at(sn, idx)), score_at(sn, idx + 1));
        mx1 = __builtin_fmaxf(__builtin_fmaxf(mx1, score_at(sn, idx + 2)), score_at(sn, idx + 3));
      }
      asm volatile("" : "+v"(mx0), "+v"(mx1));
    }
    if (i + R2 < N2) vt[i + R2] = read_vt<D, T>(vb[(i + R2) % G::DT], (i + R2) / G::DT);
    __builtin_amdgcn_sched_barrier(0);
  }
  l += ps0 + ps1;
  return fmaxf(mx0, mx1);
}

// Scores of a slot exp'd under the previous slot's PV MFMAs in the lazy mode
// (the rest run under the slot's own score MFMAs). Half and half measured
// fastest at D = 128: 8, 12, 20 and 24 (24 spills) were 0.3-1.9 % slower.
#ifndef TTCD_EA
#define TTCD_EA 16
#endif
template <int D>
constexpr int lazy_ea() {
  return TTCD_EA;
}

// exp2 of score idx of s against mc, packed in pairs into P^T k-step idx / 8
// of p, summed in idx order (even / odd chains, as the exact mode sums them).
template <typename T>
__device__ __forceinline__ void exp_one(const f32x16 (&s)[2], typename VecT<T>::v8 (&p)[4],
                                        int idx, float c, float mc, float& pe, float& ps0,
                                        float& ps1) {
  const float v = fast_exp2(fmaf(score_at(s, idx), c, -mc));
  if (idx & 1) {
    p[idx >> 3][(idx & 7) - 1] = static_cast<T>(pe);
    p[idx >> 3][idx & 7] = static_cast<T>(v);
    ps1 = idx == 1 ? v : ps1 + v;
  } else {
    pe = v;
    ps0 = idx == 0 ? v : ps0 + v;
  }
}

// The slot of the lazy mode (rescale_log2 > 0). Each row keeps its reference
// max m until a slot's probabilities against it leave the bound: the slot's
// sum of p over a half-row (32 keys) exceeds 2^rescale_log2 (so every p stays
// <= 2^rescale_log2, the exact mode's bound), or the row has no reference
// yet. No row max is taken in the common path: rescue() takes it in the rare
// slot that crosses the bound, and that slot's exp2 are redone against the
// new reference. The exp2 of a slot need no max first, so they are split
// over two slots' MFMAs. Issue order:
//   phase 1: the scores S(k+1) (2*DK MFMAs), K operand reads R1 ahead, with
//            the exp2 / packing / row sums of S(k) scores EA .. 31 between
//            them (scores 0 .. EA-1 ran in the previous slot).
//   check:   rescue(lane sum, mc): one compare and a wave-uniform branch in
//            the common path. It moves the references of the rows out of
//            bound, rescales O^T and l, and returns true if S(k) must be
//            redone; then l += the slot's sums.
//   phase 2: PV(k) (4*DT MFMAs) from pc, V^T reads R2 ahead, with the exp2 of
//            S(k+1) scores 0 .. EA-1 into pn, against pre_next() (which masks
//            S(k+1) if needed and returns its m*c, +inf for a skipped slot).
// mc and ps0 / ps1 / pe carry the next slot's exp2 state across the call.
template <int D, typename T, typename PreNext, typename Rescue>
__device__ __forceinline__ void slot_body_lazy(const Ctx<D, T>& x, f32x16 (&sc)[2],
                                               f32x16 (&sn)[2], typename VecT<T>::v8 (&pc)[4],
                                               typename VecT<T>::v8 (&pn)[4],
                                               f32x16 (&o)[Geo<D>::DT], float& l, float& mc,
                                               float& ps0, float& ps1, float& pe,
                                               const LDS_AS char* kb, const LDS_AS char* vbase,
                                               PreNext&& pre_next, Rescue&& rescue) {
  using G = Geo<D>;
  using v8 = typename VecT<T>::v8;
  constexpr int N1 = 2 * G::DK;
  constexpr int N2 = 4 * G::DT;
  constexpr int R1 = TTCD_R1;
  constexpr int R2 = TTCD_R2;
  constexpr int EA = lazy_ea<D>();
  static_assert(EA >= 0 && EA <= 32, "scores per phase");

  // The K lane address is opaque per slot, so its eight per-k-step XORs are
  // formed here instead of held in registers. The V^T addresses need no such
  // fence (their per-k-step parts are immediate offsets); one costs four
  // register copies per slot and, at this register budget, a spill.
  uint32_t xk = x.ln.xk;
  asm volatile("" : "+v"(xk));
  const LDS_AS char* vb[G::DT];
#pragma unroll
  for (int dt = 0; dt < G::DT; ++dt) vb[dt] = vbase + x.ln.vb[dt];

  // phase 1
  v8 ka[N1];
#pragma unroll
  for (int i = 0; i < R1; ++i) ka[i] = read_k<D, T>(kb, xk, i);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < N1; ++i) {
    const int kt = i & 1, ks = i >> 1;
    sn[kt] = mfma32(ka[i], x.qf[ks], i < 2 ? f32x16{} : sn[kt]);
    if (i + R1 < N1) ka[i + R1] = read_k<D, T>(kb, xk, i + R1);
    const int e0 = EA + (32 - EA) * i / N1, e1 = EA + (32 - EA) * (i + 1) / N1;
#pragma unroll
    for (int idx = e0; idx < e1; ++idx) exp_one<T>(sc, pc, idx, x.c, mc, pe, ps0, ps1);
    // keep the sums here, in the MFMA shadow (otherwise they sink to the check)
    asm volatile("" : "+v"(ps0), "+v"(ps1));
    __builtin_amdgcn_sched_barrier(0);
  }

  if (__builtin_expect(rescue(ps0 + ps1, mc), 0)) {
#pragma unroll
    for (int idx = 0; idx < 32; ++idx) exp_one<T>(sc, pc, idx, x.c, mc, pe, ps0, ps1);
  }
  l += ps0 + ps1;
  mc = pre_next();
  ps0 = ps1 = 0.f;

  // phase 2
  v8 vt[N2];
#pragma unroll
  for (int i = 0; i < R2; ++i) vt[i] = read_vt<D, T>(vb[i % G::DT], i / G::DT);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < N2; ++i) {
    const int ks = i / G::DT, dt = i % G::DT;
    o[dt] = mfma32(vt[i], pc[ks], o[dt]);
    const int e0 = EA * i / N2, e1 = EA * (i + 1) / N2;
#pragma unroll
    for (int idx = e0; idx < e1; ++idx) exp_one<T>(sn, pn, idx, x.c, mc, pe, ps0, ps1);
    asm volatile("" : "+v"(ps0), "+v"(ps1));
    if (i + R2 < N2) vt[i + R2] = read_vt<D, T>(vb[(i + R2) % G::DT], (i + R2) / G::DT);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// A wave-uniform 64-bit pointer held in scalar registers.
template <typename T>
__device__ __forceinline__ const T* uniform_ptr(const T* p) {
  const uint64_t b = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  return reinterpret_cast<const T*>((uint64_t)lo | ((uint64_t)hi << 32));
}

// Wavefronts per SIMD: two for D = 128 (<= 256 VGPRs); three for D = 64, whose
// slots carry half the MFMA work for the same softmax VALU work and need
// more waves to issue from (<= 168 VGPRs, 3 x 32 KiB of LDS per CU).
#ifndef TTCD_D64_WAVES
#define TTCD_D64_WAVES 3
#endif
template <int D>
constexpr int waves_per_simd() {
  return D == 64 ? TTCD_D64_WAVES : 2;
}

template <int D, typename T, bool DUAL, bool LAZY>
__global__ __attribute__((amdgpu_flat_work_group_size(kWaves * 64, kWaves * 64),
                          amdgpu_waves_per_eu(waves_per_simd<D>(), waves_per_simd<D>())))
void attn_fwd_kernel(AttnArgs a) {
  using G = Geo<D>;
  using v8 = typename VecT<T>::v8;
  __shared__ __attribute__((aligned(1024))) char smem_raw[G::NSTAGE * G::STAGE_B];

  const int tid = __builtin_amdgcn_workitem_id_x();
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Wavefront geometry: R query rows per wavefront, 32 of one head or (hpw =
  // 2, even GQA group) 16 of each of two heads of the group; score column
  // n = lane % 32 is row n % R of head h + n / R.
  const int R = a.sched.rows;
  const int hpw = kWaveRows / R;
  const int span = kWaves * R;
  // Workgroup -> (b, kv head, query block [heaviest first], head group),
  // XCD-remapped: each XCD sweeps a contiguous run, so the query heads
  // sharing a K/V head and neighbouring query blocks share its L2.
  int rest = xcd_remap(__builtin_amdgcn_workgroup_id_x(), a.nwg);
  const int ngrp = a.G / hpw;
  const int g = rest % ngrp;
  rest /= ngrp;
  const int qb = a.qb0 + (a.nqb - 1 - rest % a.nqb);
  rest /= a.nqb;
  const int hk = rest % a.Hkv;
  const int b = rest / a.Hkv;
  const int h = hk * a.G + g * hpw;  // the wavefront's first query head
  // this lane's head is h + dh (kept out of the uniform bases below, so they
  // stay in scalar registers through the sweep)
  const bool dh = hpw == 2 && ((lane >> 4) & 1) != 0;
  const int t0 = qb * span;

  // Packed sequences: sequence b is rows row0 .. row0 + T_ - 1 of every
  // tensor, with its own schedule. The bounds are clamped to the packed
  // tensors and to the launched query blocks, so no cu_seqlens value can
  // move an access out of them; a workgroup past its sequence's end leaves
  // before its first barrier.
  int T_ = a.T;
  int64_t row0 = 0;
  Schedule sc = a.sched;
  if (a.cu_seqlens != nullptr) {
    const int c0 = __builtin_amdgcn_readfirstlane(a.cu_seqlens[b]);
    const int c1 = __builtin_amdgcn_readfirstlane(a.cu_seqlens[b + 1]);
    const int s0 = min(max(c0, 0), a.total);
    const int s1 = min(max(c1, s0), a.total);
    T_ = min(s1 - s0, a.nqb * span);
    row0 = s0;
    sc = sc.dual ? make_dual_schedule(T_, a.win_a, a.win_b, R)
                 : make_band_schedule(T_, a.win_a, a.win_b, R);
    if (t0 >= T_) return;
  }
  const int r0 = __builtin_amdgcn_readfirstlane(t0 + wave * R);
  const int t_last = min(t0 + span, T_) - 1;
  const int q_off = a.q_off;
  // a wave with no row in [q_off, T) computes nothing (it still takes part
  // in the workgroup's loads and barriers)
  const bool wave_valid = (r0 < T_) & (r0 + R > q_off);

  const T* qp =
      static_cast<const T*>(a.q) + b * a.q_sb + (h + dh) * a.q_sh + row0 * a.q_st;
  const T* kp =
      uniform_ptr(static_cast<const T*>(a.k) + b * a.k_sb + hk * a.k_sh + row0 * a.k_st);
  const T* vp =
      uniform_ptr(static_cast<const T*>(a.v) + b * a.v_sb + hk * a.v_sh + row0 * a.v_st);
  // first output row / LSE entry of this (b, h); the lane's own head adds
  // o_dh / lse_dh
  const int64_t o_base = b * a.o_sb + h * a.o_sh + row0 * a.o_st;
  const int64_t lse_base = b * a.lse_sb + h * a.lse_sh + row0;
  auto o_dh = [&]() __attribute__((always_inline)) { return dh ? a.o_sh : (int64_t)0; };
  auto lse_dh = [&]() __attribute__((always_inline)) { return dh ? a.lse_sh : (int64_t)0; };

  Ctx<D, T> x;
  x.lds = (LDS_AS char*)smem_raw;
  const uint32_t lds_base = (uint32_t)(uintptr_t)x.lds;
  x.c = a.c;
  x.qrow = r0 + (lane & (R - 1));
  x.half = lane >> 5;
  x.T_ = T_;
  x.ln = make_lane<D>(a.k_st, a.v_st, wave, lane);
  {
    const bool row_ok = (x.qrow < T_) & (x.qrow >= q_off);
    const T* src = qp + (int64_t)(row_ok ? x.qrow - q_off : 0) * a.q_st + (lane >> 5) * 8;
#pragma unroll
    for (int ks = 0; ks < G::DK; ++ks) {
      v8 z = {};
      x.qf[ks] = row_ok ? *reinterpret_cast<const v8*>(src + ks * 16) : z;
    }
  }

  int n_hi = 0, n_lo = 1;
  if (!sc.wg_range(t0, t_last, &n_hi, &n_lo)) {
    n_hi = 0;
    n_lo = 1;
  }
  const int count = n_hi - n_lo + 1;
  const SlotPlan sp = make_slot_plan(
      sc, [&](int wv) { return t0 + wv * R; }, n_hi, n_lo);
  // The plan is workgroup-uniform; keep it in scalar registers.
  const int nslot = __builtin_amdgcn_readfirstlane(count > 0 ? sp.slots() : 0);

  const WaveSlots wsl(sc, r0);
  const int64_t kst = a.k_st, vst = a.v_st;
  const float rescale_log2 = a.rescale_log2;
  // Byte address of tile 0's first key (key -kshift) and bytes per key: an
  // interior tile's address is then one 32 x 32 -> 64-bit product with
  // (word & ~63) = 64 n (token strides are below 2^25 elements).
  const uint64_t k_tile0 =
      reinterpret_cast<uint64_t>(kp) - (uint64_t)((int64_t)sc.kshift * kst * 2);
  const uint64_t v_tile0 =
      reinterpret_cast<uint64_t>(vp) - (uint64_t)((int64_t)sc.kshift * vst * 2);
  const uint32_t k_row_b = (uint32_t)(kst * 2), v_row_b = (uint32_t)(vst * 2);
  // DMA of the K (or V) tile of the slot with word w into the K (V) half of
  // stage s; nothing for a word past the last slot.
  auto dma_half = [&](bool is_k, uint32_t w, int s) __attribute__((always_inline)) {
    const uint32_t dst = lds_base + s * G::STAGE_B + (is_k ? 0 : G::TILE_B);
    const uint32_t(&off)[G::NDMA] = is_k ? x.ln.k_off : x.ln.v_off;
    if (__builtin_expect((w & kWordInterior) != 0, 1)) {
      const uint64_t tile =
          (is_k ? k_tile0 : v_tile0) + (uint64_t)(w & ~63u) * (is_k ? k_row_b : v_row_b);
      dma_run<G::NDMA>(reinterpret_cast<const void*>(tile), off, dst + wave * 1024);
    } else if (w & kWordLoad) {
      if (is_k)
        dma_tile<D, T, true>(dst, kp, kst, word_j0(sc, w), T_, wave, lane, off, false);
      else
        dma_tile<D, T, false>(dst, vp, vst, word_j0(sc, w), T_, wave, lane, off, false);
    }
  };

  f32x16 o[G::DT];
#pragma unroll
  for (int dt = 0; dt < G::DT; ++dt) o[dt] = f32x16{};
  float m = -INFINITY, l = 0.f;
  float mc_ref = 0.f;  // lazy mode: m*c, 0 while the row has no reference
  const float bound = LAZY ? exp2f(a.rescale_log2) : 0.f;
  bool emitted_s = false;
  f32x16 s0[2], s1[2];
  // lazy mode: P^T of two consecutive slots, and the exp2 state carried from
  // a slot's PV phase into the next slot
  v8 pa[4], pb[4];
  float lz_mc = 0.f, lz_ps0 = 0.f, lz_ps1 = 0.f, lz_pe = 0.f;

  // Two stages; stage k % 2 holds K(k) and V(k). In slot k the scores read
  // K(k+1) and PV reads V(k), so K(k+2) can replace K(k) (read in slot k-1)
  // and V(k+1) can replace V(k-1): both are fetched at the start of slot k
  // and have the whole slot to land.
  // Slot words (schedule.h: slot_word) of this wave for slots tb .. tb+63,
  // slot tb + lane in each lane; refreshed every 64 slots and read back one
  // slot at a time with v_readlane.
  auto words = [&](int tb) __attribute__((always_inline)) {
    return slot_word(sc, sp, wsl, nslot, wave_valid, T_, tb + lane);
  };
  uint32_t tbl = words(0);
  // Prologue: K(0), V(0), K(1) in LDS, scores of slot 0. w_cur and w_nxt are
  // the words of slots 0 and 1.
  uint32_t w_cur = (uint32_t)__builtin_amdgcn_readlane((int)tbl, 0);
  uint32_t w_nxt = (uint32_t)__builtin_amdgcn_readlane((int)tbl, 1);
  dma_half(true, w_cur, 0);
  dma_half(false, w_cur, 0);
  dma_half(true, w_nxt, 1);
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  // Scores of slot 0 and their lane max (unmasked; slot 0's mask and
  // reference max are settled inside the first slot).
  float mx_lane = -INFINITY;
  {
    s0[0] = f32x16{};
    s0[1] = f32x16{};
#pragma unroll
    for (int i = 0; i < 2 * G::DK; ++i)
      s0[i & 1] = mfma32(read_k<D, T>(x.lds, x.ln.xk, i), x.qf[i >> 1], s0[i & 1]);
    if constexpr (!LAZY) {
      float a0 = -INFINITY, a1 = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        a0 = fmaxf(a0, s0[0][e]);
        a1 = fmaxf(a1, s0[1][e]);
      }
      mx_lane = fmaxf(a0, a1);
    }
  }
  if constexpr (LAZY) {
    // slot 0's first exp2 (the later slots' run under the previous PV)
    if (__builtin_expect((w_cur & kWordMask) != 0, 0))
      mask_band(s0, x.qrow, word_j0(sc, w_cur), T_, word_band(sc, w_cur), x.half);
    lz_mc = (w_cur & kWordActive) ? mc_ref : INFINITY;
#pragma unroll
    for (int idx = 0; idx < lazy_ea<D>(); ++idx)
      exp_one<T>(s0, pa, idx, x.c, lz_mc, lz_pe, lz_ps0, lz_ps1);
  }
  // every wave has read K(0) before slot 0 replaces it with K(2)
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // Slot k: the scores of slot k are in scur (lane max mx_lane, not yet
  // masked); fold them and compute the scores of slot k+1 into snxt. Every
  // slot runs the same code: a slot this wave skips folds all-zero
  // probabilities. Unrolled by two so the two score buffers swap roles
  // without register copies.
  auto step = [&](f32x16 (&scur)[2], f32x16 (&snxt)[2], v8 (&pcur)[4], v8 (&pnxt)[4], int k)
                  __attribute__((always_inline)) {
    const int k2 = k + 2;
    if (__builtin_expect((k2 & 63) == 0, 0)) tbl = words(k2);
    const uint32_t w_k2 = (uint32_t)__builtin_amdgcn_readlane((int)tbl, k2 & 63);
    dma_half(true, w_k2, k & 1);
    dma_half(false, w_nxt, (k + 1) & 1);
    // Mask S(k) if needed, then the reference max of slot k (lazy rescale):
    // moved, and O^T / l rescaled, only when some row's max exceeds it by
    // more than 2^rescale_log2 (0: whenever it grows, the reference kernel's
    // exact running max). Returns m*c for the exp2 of slot k.
    auto settle = [&]() __attribute__((always_inline)) {
      float mx = mx_lane;
      if (__builtin_expect((w_cur & kWordMask) != 0, 0)) {
        mask_band(scur, x.qrow, word_j0(sc, w_cur), T_, word_band(sc, w_cur), x.half);
        float a0 = -INFINITY, a1 = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          a0 = fmaxf(a0, scur[0][e]);
          a1 = fmaxf(a1, scur[1][e]);
        }
        mx = fmaxf(a0, a1);
      }
      mx = xhalf_max(mx);
      const bool active = (w_cur & kWordActive) != 0;
      const float m_new = active ? fmaxf(m, mx) : m;
      const bool grow = (m_new > m) & ((m == -INFINITY) | ((m_new - m) * x.c > rescale_log2));
      if (__builtin_expect(__any(grow) != 0, 0)) {
        // Only the lanes past the threshold move their reference max (the
        // others keep theirs, alpha = 1), so every row's arithmetic depends
        // on its own scores alone, not on the other rows of its wavefront.
        const float m_set = grow ? m_new : m;
        const float mc_new = (m_set == -INFINITY) ? 0.f : m_set * x.c;
        const float alpha = grow ? fast_exp2(fmaf(m, x.c, -mc_new)) : 1.f;
        l *= alpha;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) o[dt] *= alpha;
        m = m_set;
      }
      return active ? ((m == -INFINITY) ? 0.f : m * x.c) : INFINITY;
    };
    const LDS_AS char* kb = x.lds + ((k + 1) & 1) * G::STAGE_B;
    const LDS_AS char* vbase = x.lds + (k & 1) * G::STAGE_B + G::TILE_B;
    if constexpr (LAZY) {
      // Mask S(k+1) if needed; m*c for its exp2 (+inf for a slot this wave
      // skips).
      auto pre_next = [&]() __attribute__((always_inline)) {
        if (__builtin_expect((w_nxt & kWordMask) != 0, 0))
          mask_band(snxt, x.qrow, word_j0(sc, w_nxt), T_, word_band(sc, w_nxt), x.half);
        return (w_nxt & kWordActive) ? mc_ref : INFINITY;
      };
      // A row is out of bound when either half's sum t exceeds 2^rescale_log2
      // or it has no reference yet. Such rows move their reference to their
      // running max (O^T and l rescaled); the others keep theirs (alpha = 1,
      // the same p), so a row's arithmetic depends on its own scores alone.
      auto rescue = [&](float t, float& mc) __attribute__((always_inline)) {
        const bool active = (w_cur & kWordActive) != 0;
        const bool out = active & (!(t <= bound) | (m == -INFINITY));
        if (__builtin_expect(__any(out) == 0, 1)) return false;
        float a0 = -INFINITY, a1 = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          a0 = fmaxf(a0, scur[0][e]);
          a1 = fmaxf(a1, scur[1][e]);
        }
        const float mx = xhalf_max(fmaxf(a0, a1));
        const bool row_out = xhalf_any(out);
        const float m_new = row_out ? fmaxf(m, mx) : m;
        const bool grow = m_new > m;
        const float mc_new = grow ? m_new * x.c : mc_ref;
        const float alpha = grow ? fast_exp2(fmaf(m, x.c, -mc_new)) : 1.f;
        l *= alpha;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) o[dt] *= alpha;
        m = grow ? m_new : m;
        mc_ref = mc_new;
        mc = mc_ref;
        return true;
      };
      slot_body_lazy<D, T>(x, scur, snxt, pcur, pnxt, o, l, lz_mc, lz_ps0, lz_ps1, lz_pe, kb,
                           vbase, pre_next, rescue);
    } else {
      mx_lane = slot_body<D, T>(x, scur, snxt, o, l, kb, vbase, settle);
    }
    if (DUAL && (w_cur & kWordLast)) {
      T* os = static_cast<T*>(a.o_s) + o_base + o_dh();
      float* lse_s = a.lse_s ? a.lse_s + lse_base + lse_dh() : nullptr;
      emit<D, T>(o, m, l, x.c, os, a.o_st, lse_s, x.qrow, T_, q_off, lane);
      emitted_s = true;
    }
    w_cur = w_nxt;
    w_nxt = w_k2;
    // K(k+2) and V(k+1), fetched at the start of this slot, are read in the next.
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  };

  for (int k = 0; k < nslot; k += 2) {
    step(s0, s1, pa, pb, k);
    if (k + 1 < nslot) step(s1, s0, pb, pa, k + 1);
  }

  if (wave_valid) {
    if (DUAL && !emitted_s) {
      T* os = static_cast<T*>(a.o_s) + o_base + o_dh();
      float* lse_s = a.lse_s ? a.lse_s + lse_base + lse_dh() : nullptr;
      emit<D, T>(o, m, l, x.c, os, a.o_st, lse_s, x.qrow, T_, q_off, lane);
    }
    T* ot = static_cast<T*>(a.o_t) + o_base + o_dh();
    float* lse_t = a.lse_t ? a.lse_t + lse_base + lse_dh() : nullptr;
    emit<D, T>(o, m, l, x.c, ot, a.o_st, lse_t, x.qrow, T_, q_off, lane);
  }
}

template <int D, typename T, bool DUAL>
hipError_t launch_typed(const AttnArgs& a, hipStream_t stream) {
  AttnArgs args = a;
  args.nwg = a.B * (a.Hq / (kWaveRows / a.sched.rows)) * a.nqb;
  // The sum-triggered lazy slot needs a second P^T buffer, which D = 64 has
  // no registers for at three waves per SIMD; D = 64 and the exact mode take
  // the max-first slot.
  if constexpr (D == 128) {
    if (a.rescale_log2 > 0.f) {
      hipLaunchKernelGGL((attn_fwd_kernel<D, T, DUAL, true>), dim3(args.nwg), dim3(kWaves * 64),
                         0, stream, args);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((attn_fwd_kernel<D, T, DUAL, false>), dim3(args.nwg), dim3(kWaves * 64), 0,
                     stream, args);
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
