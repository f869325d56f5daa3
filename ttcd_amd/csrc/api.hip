// api.hip - the extern "C" entry points declared in include/ttcd.h:
// argument validation (before any HIP call, so every error path is
// testable without a GPU), status/error reporting, and the host replay of
// the attention schedule used by the coverage tests.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>

#include "internal.h"
#include "schedule.h"
#include "ttcd.h"

namespace {

thread_local char g_err[512] = "";

ttcd_status fail(ttcd_status st, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return st;
}

ttcd_status ok() {
  g_err[0] = '\0';
  return TTCD_OK;
}

ttcd_status from_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(TTCD_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Largest K/V token stride (elements) the tile loads' 32-bit lane offsets reach.
constexpr int64_t kMaxTokenStride = int64_t(1) << 25;

// Checks shared by both attention entry points.
ttcd_status check_attn(const void* q, const void* k, const void* v, const void* o, int B, int T,
                       int Hq, int Hkv, int D, const int64_t* qs, const int64_t* ks,
                       const int64_t* vs, const int64_t* os, ttcd_dtype dtype) {
  if (!q || !k || !v || !o) return fail(TTCD_ERR_INVALID_ARGUMENT, "null tensor pointer");
  if (!qs || !ks || !vs || !os) return fail(TTCD_ERR_INVALID_ARGUMENT, "null stride array");
  if (B < 1 || T < 1 || Hq < 1 || Hkv < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "B, T, Hq, Hkv must be >= 1 (got %d, %d, %d, %d)", B,
                T, Hq, Hkv);
  if (Hq % Hkv != 0)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "Hq (%d) must be a multiple of Hkv (%d)", Hq, Hkv);
  if (D != 64 && D != 128)
    return fail(TTCD_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", D);
  if (dtype != TTCD_DTYPE_BF16 && dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "attention dtype must be bf16 or f16");
  if (qs[3] != 1 || ks[3] != 1 || vs[3] != 1 || os[3] != 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "head_dim must be contiguous (d-stride 1)");
  const int64_t* all[4] = {qs, ks, vs, os};
  for (int t = 0; t < 4; ++t)
    for (int i = 0; i < 3; ++i)
      if (all[t][i] % 8 != 0 || all[t][i] < 0)
        return fail(TTCD_ERR_UNSUPPORTED,
                    "strides must be non-negative multiples of 8 elements (16-byte rows)");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(TTCD_ERR_UNSUPPORTED, "tensor base pointers must be 16-byte aligned");
  // The K/V tile loads address a lane's chunk with a 32-bit byte offset from the
  // tile's first key: 63 token strides of 2-byte elements plus one row must fit.
  if (ks[1] > kMaxTokenStride || vs[1] > kMaxTokenStride)
    return fail(TTCD_ERR_UNSUPPORTED, "k/v token stride above %lld elements",
                (long long)kMaxTokenStride);
  const int64_t nqb = (T + ttcd::kBlockM - 1) / ttcd::kBlockM;
  if ((int64_t)B * Hq * nqb > 0x7fffffffLL)  // bound on workgroups for either geometry
    return fail(TTCD_ERR_UNSUPPORTED, "grid too large");
  return TTCD_OK;
}

// The lazy-rescale threshold: finite, 0 (exact running max) .. 16. Every
// probability p = exp2(s*c - m*c) stays <= 2^rescale_log2 and is rounded to
// the input dtype before PV: bf16 holds any such p, but f16 rounds values
// >= 65520 to +inf, so F16 is limited to 15 (p <= 32768).
ttcd_status check_rescale(float rescale_log2, ttcd_dtype dtype) {
  const float hi = dtype == TTCD_DTYPE_F16 ? 15.f : 16.f;
  if (!(rescale_log2 >= 0.f && rescale_log2 <= hi))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "rescale_log2 must be in [0, %g] for this dtype (got %g)",
                (double)hi, (double)rescale_log2);
  return TTCD_OK;
}

ttcd::AttnArgs fill_args(const void* q, const void* k, const void* v, int B, int T, int Hq,
                         int Hkv, const int64_t* qs, const int64_t* ks, const int64_t* vs,
                         const int64_t* os, float sm_scale) {
  ttcd::AttnArgs a = {};
  a.q = q;
  a.k = k;
  a.v = v;
  a.q_sb = qs[0];
  a.q_st = qs[1];
  a.q_sh = qs[2];
  a.k_sb = ks[0];
  a.k_st = ks[1];
  a.k_sh = ks[2];
  a.v_sb = vs[0];
  a.v_st = vs[1];
  a.v_sh = vs[2];
  a.o_sb = os[0];
  a.o_st = os[1];
  a.o_sh = os[2];
  a.B = B;
  a.T = T;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  const int span = ttcd::wg_span_tokens(a.G);
  a.q_off = 0;
  a.qb0 = 0;
  a.nqb = (T + span - 1) / span;  // query blocks per (b, slice)
  a.c = sm_scale * 1.4426950408889634f;
  return a;
}

ttcd::Elem elem(ttcd_dtype d) {
  return d == TTCD_DTYPE_BF16 ? ttcd::Elem::BF16
                              : (d == TTCD_DTYPE_F16 ? ttcd::Elem::F16 : ttcd::Elem::F32);
}

}  // namespace

extern "C" {

const char* ttcd_status_string(ttcd_status status) {
  switch (status) {
    case TTCD_OK: return "TTCD_OK";
    case TTCD_ERR_INVALID_ARGUMENT: return "TTCD_ERR_INVALID_ARGUMENT";
    case TTCD_ERR_UNSUPPORTED: return "TTCD_ERR_UNSUPPORTED";
    case TTCD_ERR_HIP: return "TTCD_ERR_HIP";
  }
  return "TTCD_ERR_UNKNOWN";
}

const char* ttcd_last_error(void) { return g_err; }

int ttcd_abi_version(void) { return TTCD_ABI_VERSION; }

// Tq query rows at absolute positions Tk - Tq .. Tk - 1 against Tk keys
// (flash-attention's bottom-right aligned causal mask); q / o are (B, Tq, ...),
// k / v (B, Tk, ...), lse (B, Hq, Tq).
static ttcd_status set_rows(ttcd::AttnArgs* a, int Tq, int Tk) {
  if (Tq < 1 || Tq > Tk)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "need 1 <= Tq <= Tk (got Tq=%d, Tk=%d)", Tq, Tk);
  const int span = ttcd::wg_span_tokens(a->G);
  a->q_off = Tk - Tq;
  a->qb0 = a->q_off / span;
  a->nqb = (Tk + span - 1) / span - a->qb0;
  a->lse_sh = Tq;
  a->lse_sb = (int64_t)a->Hq * Tq;
  return TTCD_OK;
}

ttcd_status ttcd_dual_window_attn_kv_fwd(const void* q, const void* k, const void* v, void* o_t,
                                         void* o_s, float* lse_t, float* lse_s, int B, int Tq,
                                         int Tk, int Hq, int Hkv, int D,
                                         const int64_t q_stride[4], const int64_t k_stride[4],
                                         const int64_t v_stride[4], const int64_t o_stride[4],
                                         int window_t, int window_s, float sm_scale,
                                         float rescale_log2, ttcd_dtype dtype, void* stream) {
  ttcd_status st =
      check_attn(q, k, v, o_t, B, Tk, Hq, Hkv, D, q_stride, k_stride, v_stride, o_stride, dtype);
  if (st == TTCD_OK) st = check_rescale(rescale_log2, dtype);
  if (st != TTCD_OK) return st;
  if (!o_s) return fail(TTCD_ERR_INVALID_ARGUMENT, "null student output pointer");
  if (!aligned16(o_s)) return fail(TTCD_ERR_UNSUPPORTED, "o_s must be 16-byte aligned");
  if (window_t < 0) window_t = Tk;
  if (window_s < 1) return fail(TTCD_ERR_INVALID_ARGUMENT, "window_s must be >= 1 (got %d)", window_s);
  if (window_s > window_t)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "window_s (%d) must be <= window_t (%d)", window_s,
                window_t);
  if (!(sm_scale > 0.f) || !isfinite(sm_scale))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "sm_scale must be finite and > 0");
  ttcd::AttnArgs a = fill_args(q, k, v, B, Tk, Hq, Hkv, q_stride, k_stride, v_stride, o_stride,
                               sm_scale);
  st = set_rows(&a, Tq, Tk);
  if (st != TTCD_OK) return st;
  a.o_t = o_t;
  a.o_s = o_s;
  a.lse_t = lse_t;
  a.lse_s = lse_s;
  a.rescale_log2 = rescale_log2;
  a.sched = ttcd::make_dual_schedule(Tk, window_s, window_t, ttcd::wave_rows(a.G));
  return from_hip(ttcd::launch_attn(a, D, elem(dtype), static_cast<hipStream_t>(stream)),
                  "dual-window attention launch");
}

ttcd_status ttcd_dual_window_attn_fwd(const void* q, const void* k, const void* v, void* o_t,
                                      void* o_s, float* lse_t, float* lse_s, int B, int T,
                                      int Hq, int Hkv, int D, const int64_t q_stride[4],
                                      const int64_t k_stride[4], const int64_t v_stride[4],
                                      const int64_t o_stride[4], int window_t, int window_s,
                                      float sm_scale, ttcd_dtype dtype, void* stream) {
  return ttcd_dual_window_attn_kv_fwd(q, k, v, o_t, o_s, lse_t, lse_s, B, T, T, Hq, Hkv, D,
                                      q_stride, k_stride, v_stride, o_stride, window_t, window_s,
                                      sm_scale, ttcd::kDefaultRescaleLog2, dtype, stream);
}

ttcd_status ttcd_band_attn_kv_fwd(const void* q, const void* k, const void* v, void* o,
                                  float* lse, int B, int Tq, int Tk, int Hq, int Hkv, int D,
                                  const int64_t q_stride[4], const int64_t k_stride[4],
                                  const int64_t v_stride[4], const int64_t o_stride[4],
                                  int band_lo, int band_hi, float sm_scale, float rescale_log2,
                                  ttcd_dtype dtype, void* stream) {
  ttcd_status st =
      check_attn(q, k, v, o, B, Tk, Hq, Hkv, D, q_stride, k_stride, v_stride, o_stride, dtype);
  if (st == TTCD_OK) st = check_rescale(rescale_log2, dtype);
  if (st != TTCD_OK) return st;
  if (band_lo < 0 || band_hi <= band_lo)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "need 0 <= band_lo < band_hi (got %d, %d)", band_lo,
                band_hi);
  if (!(sm_scale > 0.f) || !isfinite(sm_scale))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "sm_scale must be finite and > 0");
  ttcd::AttnArgs a = fill_args(q, k, v, B, Tk, Hq, Hkv, q_stride, k_stride, v_stride, o_stride,
                               sm_scale);
  st = set_rows(&a, Tq, Tk);
  if (st != TTCD_OK) return st;
  a.o_t = o;
  a.lse_t = lse;
  a.rescale_log2 = rescale_log2;
  a.sched = ttcd::make_band_schedule(Tk, band_lo, band_hi, ttcd::wave_rows(a.G));
  return from_hip(ttcd::launch_attn(a, D, elem(dtype), static_cast<hipStream_t>(stream)),
                  "band attention launch");
}

ttcd_status ttcd_band_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                               int B, int T, int Hq, int Hkv, int D, const int64_t q_stride[4],
                               const int64_t k_stride[4], const int64_t v_stride[4],
                               const int64_t o_stride[4], int band_lo, int band_hi,
                               float sm_scale, ttcd_dtype dtype, void* stream) {
  return ttcd_band_attn_kv_fwd(q, k, v, o, lse, B, T, T, Hq, Hkv, D, q_stride, k_stride,
                               v_stride, o_stride, band_lo, band_hi, sm_scale,
                               ttcd::kDefaultRescaleLog2, dtype, stream);
}

// Packed sequences (flash-attention's varlen layout): q / o are (total, Hq, D),
// k / v (total, Hkv, D), LSEs (Hq, total); sequence b is rows
// cu_seqlens[b] .. cu_seqlens[b+1]-1. The kernel reads cu_seqlens on the
// device (no host sync) and clamps every sequence to [0, total) and to
// max_seqlen rows, so malformed offsets cannot move an access out of the
// tensors; rows outside every sequence are not written.
static ttcd_status varlen_args(ttcd::AttnArgs* a, const void* q, const void* k, const void* v,
                               const void* o, const int32_t* cu_seqlens, int nseq,
                               int max_seqlen, int total, int Hq, int Hkv, int D,
                               const int64_t* qs3, const int64_t* ks3, const int64_t* vs3,
                               const int64_t* os3, float sm_scale, float rescale_log2,
                               ttcd_dtype dtype) {
  if (!cu_seqlens) return fail(TTCD_ERR_INVALID_ARGUMENT, "null cu_seqlens");
  if (check_rescale(rescale_log2, dtype) != TTCD_OK) return TTCD_ERR_INVALID_ARGUMENT;
  if (!qs3 || !ks3 || !vs3 || !os3) return fail(TTCD_ERR_INVALID_ARGUMENT, "null stride array");
  if (nseq < 1 || max_seqlen < 1 || total < 0)
    return fail(TTCD_ERR_INVALID_ARGUMENT,
                "need nseq >= 1, max_seqlen >= 1, total >= 0 (got %d, %d, %d)", nseq, max_seqlen,
                total);
  if (!(sm_scale > 0.f) || !isfinite(sm_scale))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "sm_scale must be finite and > 0");
  const int64_t qs[4] = {0, qs3[0], qs3[1], qs3[2]}, ks[4] = {0, ks3[0], ks3[1], ks3[2]};
  const int64_t vs[4] = {0, vs3[0], vs3[1], vs3[2]}, os[4] = {0, os3[0], os3[1], os3[2]};
  ttcd_status st = check_attn(q, k, v, o, nseq, max_seqlen, Hq, Hkv, D, qs, ks, vs, os, dtype);
  if (st != TTCD_OK) return st;
  *a = fill_args(q, k, v, nseq, max_seqlen, Hq, Hkv, qs, ks, vs, os, sm_scale);
  a->cu_seqlens = cu_seqlens;
  a->total = total;
  a->lse_sb = 0;
  a->lse_sh = total;
  a->rescale_log2 = rescale_log2;
  return TTCD_OK;
}

ttcd_status ttcd_dual_window_attn_varlen_fwd(const void* q, const void* k, const void* v,
                                             void* o_t, void* o_s, float* lse_t, float* lse_s,
                                             const int32_t* cu_seqlens, int nseq, int max_seqlen,
                                             int total, int Hq, int Hkv, int D,
                                             const int64_t q_stride[3],
                                             const int64_t k_stride[3],
                                             const int64_t v_stride[3],
                                             const int64_t o_stride[3], int window_t,
                                             int window_s, float sm_scale, float rescale_log2,
                                             ttcd_dtype dtype, void* stream) {
  ttcd::AttnArgs a;
  ttcd_status st = varlen_args(&a, q, k, v, o_t, cu_seqlens, nseq, max_seqlen, total, Hq, Hkv,
                               D, q_stride, k_stride, v_stride, o_stride, sm_scale, rescale_log2,
                               dtype);
  if (st != TTCD_OK) return st;
  if (!o_s) return fail(TTCD_ERR_INVALID_ARGUMENT, "null student output pointer");
  if (!aligned16(o_s)) return fail(TTCD_ERR_UNSUPPORTED, "o_s must be 16-byte aligned");
  if (window_s < 1) return fail(TTCD_ERR_INVALID_ARGUMENT, "window_s must be >= 1 (got %d)", window_s);
  if (window_t >= 0 && window_s > window_t)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "window_s (%d) must be <= window_t (%d)", window_s,
                window_t);
  // full causal: a teacher window no sequence reaches (clamped to each length)
  if (window_t < 0) window_t = 0x3fffffff;
  a.o_t = o_t;
  a.o_s = o_s;
  a.lse_t = lse_t;
  a.lse_s = lse_s;
  a.win_a = window_s;
  a.win_b = window_t;
  a.sched = ttcd::make_dual_schedule(max_seqlen, window_s, window_t, ttcd::wave_rows(a.G));
  return from_hip(ttcd::launch_attn(a, D, elem(dtype), static_cast<hipStream_t>(stream)),
                  "varlen dual-window attention launch");
}

ttcd_status ttcd_band_attn_varlen_fwd(const void* q, const void* k, const void* v, void* o,
                                      float* lse, const int32_t* cu_seqlens, int nseq,
                                      int max_seqlen, int total, int Hq, int Hkv, int D,
                                      const int64_t q_stride[3], const int64_t k_stride[3],
                                      const int64_t v_stride[3], const int64_t o_stride[3],
                                      int band_lo, int band_hi, float sm_scale,
                                      float rescale_log2, ttcd_dtype dtype, void* stream) {
  ttcd::AttnArgs a;
  ttcd_status st = varlen_args(&a, q, k, v, o, cu_seqlens, nseq, max_seqlen, total, Hq, Hkv, D,
                               q_stride, k_stride, v_stride, o_stride, sm_scale, rescale_log2,
                               dtype);
  if (st != TTCD_OK) return st;
  if (band_lo < 0 || band_hi <= band_lo)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "need 0 <= band_lo < band_hi (got %d, %d)", band_lo,
                band_hi);
  a.o_t = o;
  a.lse_t = lse;
  a.win_a = band_lo;
  a.win_b = band_hi;
  a.sched = ttcd::make_band_schedule(max_seqlen, band_lo, band_hi, ttcd::wave_rows(a.G));
  return from_hip(ttcd::launch_attn(a, D, elem(dtype), static_cast<hipStream_t>(stream)),
                  "varlen band attention launch");
}

ttcd_status ttcd_lse_merge_fwd(const void* o_s, const float* lse_s, const void* o_f,
                               const float* lse_f, void* o_t, int B, int T, int H, int D,
                               int row_start, const int64_t o_stride[4], ttcd_dtype dtype,
                               void* stream) {
  if (!o_s || !lse_s || !o_f || !lse_f || !o_t || !o_stride)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (B < 1 || T < 1 || H < 1 || D < 8)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "B, T, H must be >= 1 and D >= 8");
  if (D % 8 != 0) return fail(TTCD_ERR_UNSUPPORTED, "D must be a multiple of 8");
  if (dtype != TTCD_DTYPE_BF16 && dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "merge dtype must be bf16 or f16");
  if (o_stride[3] != 1) return fail(TTCD_ERR_INVALID_ARGUMENT, "D must be contiguous");
  for (int i = 0; i < 3; ++i)
    if (o_stride[i] % 8 != 0 || o_stride[i] < 0)
      return fail(TTCD_ERR_UNSUPPORTED, "strides must be non-negative multiples of 8");
  if (!aligned16(o_s) || !aligned16(o_f) || !aligned16(o_t))
    return fail(TTCD_ERR_UNSUPPORTED, "outputs must be 16-byte aligned");
  if (row_start < 0) return fail(TTCD_ERR_INVALID_ARGUMENT, "row_start must be >= 0");
  ttcd::MergeArgs m = {o_s, lse_s, o_f, lse_f, o_t, B, T, H, D, row_start,
                       o_stride[0], o_stride[1], o_stride[2],
                       o_stride[0], o_stride[1], o_stride[2]};
  return from_hip(ttcd::launch_lse_merge(m, elem(dtype), static_cast<hipStream_t>(stream)),
                  "lse merge launch");
}

// ---------------------------------------------------------------------------
// The LSE-combination variant as one call (lse_dual_window_attn_fa3_fast,
// profiling/lse_dual_attn.py:134-160, with the cached-prefill rows of the kv
// forms). Query rows whose absolute position is below window_s have an empty
// far band: they are one student call, copied to o_t. The other rows run in
// chunks that fit the scratch: per chunk a student call (o_s rows + lse_s),
// a far-band call (o_f + lse_f) and the merge into o_t. Each row's tiles,
// order and arithmetic depend only on its absolute position, so the result
// does not depend on the chunking.
namespace {

constexpr size_t kScratchAlign = 256;
size_t align_up(size_t x) { return (x + kScratchAlign - 1) & ~(kScratchAlign - 1); }

struct LseDual {
  const void *q, *k, *v;
  void *o_t, *o_s;
  int B, Tq, Tk, Hq, Hkv, D, WT, WS;
  const int64_t *qs, *ks, *vs, *os;
  float sm_scale, rescale_log2;
  ttcd_dtype dtype;
  int esize() const { return 2; }
  // first query row with a far band (absolute position >= WS)
  int n0() const {
    const int r = WS - (Tk - Tq);
    return r < 0 ? 0 : (r > Tq ? Tq : r);
  }
  // scratch of a chunk of `rows` rows: o_f (B, rows, Hq, D), lse_s and lse_f (B, Hq, rows)
  size_t chunk_bytes(int64_t rows) const {
    return align_up((size_t)B * rows * Hq * D * esize()) + 2 * align_up((size_t)B * Hq * rows * 4);
  }
  // most rows per chunk that `bytes` of scratch hold (a multiple of the
  // 128-row query block when at least one block fits); 0 if not even one row
  int64_t rows_fitting(size_t bytes) const {
    const int64_t need = Tq - n0();
    if (need <= 0) return 1;
    if (chunk_bytes(need) <= bytes) return need;
    const size_t per_row = (size_t)B * Hq * (D * esize() + 8);
    int64_t r = bytes > 3 * kScratchAlign ? (int64_t)((bytes - 3 * kScratchAlign) / per_row) : 0;
    while (r > 0 && chunk_bytes(r) > bytes) --r;
    if (r >= ttcd::kBlockM) r -= r % ttcd::kBlockM;
    return r;
  }
};

// Window and pointer checks of the LSE variant (the band calls check the rest).
ttcd_status check_lse_dual(LseDual* a, int window_t, int window_s) {
  if (!a->q || !a->k || !a->v || !a->o_t || !a->o_s)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "null tensor pointer");
  if (!a->qs || !a->ks || !a->vs || !a->os)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "null stride array");
  if (a->B < 1 || a->Tq < 1 || a->Tq > a->Tk || a->Hq < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "need B >= 1, Hq >= 1, 1 <= Tq <= Tk (got %d, %d, %d, %d)",
                a->B, a->Hq, a->Tq, a->Tk);
  if (a->dtype != TTCD_DTYPE_BF16 && a->dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "attention dtype must be bf16 or f16");
  if (window_t < 0) window_t = a->Tk;
  if (window_s < 1) return fail(TTCD_ERR_INVALID_ARGUMENT, "window_s must be >= 1 (got %d)", window_s);
  // lse_dual_attn.py:20: the far band [WS, WT) must not be empty
  if (window_s >= window_t)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "window_s (%d) must be < window_t (%d)", window_s,
                window_t);
  if (!aligned16(a->o_t) || !aligned16(a->o_s))
    return fail(TTCD_ERR_UNSUPPORTED, "outputs must be 16-byte aligned");
  // everything the band calls check, before any HIP call
  ttcd_status st = check_attn(a->q, a->k, a->v, a->o_t, a->B, a->Tk, a->Hq, a->Hkv, a->D, a->qs,
                              a->ks, a->vs, a->os, a->dtype);
  if (st == TTCD_OK) st = check_rescale(a->rescale_log2, a->dtype);
  if (!(a->sm_scale > 0.f) || !isfinite(a->sm_scale))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "sm_scale must be finite and > 0");
  if (st != TTCD_OK) return st;
  a->WT = window_t;
  a->WS = window_s;
  return TTCD_OK;
}

// Run the variant with `ws_bytes` of device scratch at `ws` (256-byte aligned).
ttcd_status run_lse_dual(const LseDual& a, char* ws, size_t ws_bytes, void* stream) {
  const int qoff = a.Tk - a.Tq, n0 = a.n0();
  const int64_t rows = a.rows_fitting(ws_bytes);
  if (n0 < a.Tq && rows < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "scratch of %zu bytes holds no query row (need %zu)",
                ws_bytes, a.chunk_bytes(1));
  const size_t es = a.esize();
  const char* q = static_cast<const char*>(a.q);
  char* o_s = static_cast<char*>(a.o_s);
  char* o_t = static_cast<char*>(a.o_t);
  const ttcd::Elem et = elem(a.dtype);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  ttcd_status st;
  if (n0 > 0) {
    // rows below WS: the student call alone; o_t = o_s
    st = ttcd_band_attn_kv_fwd(a.q, a.k, a.v, a.o_s, nullptr, a.B, n0, qoff + n0, a.Hq, a.Hkv,
                               a.D, a.qs, a.ks, a.vs, a.os, 0, a.WS, a.sm_scale, a.rescale_log2,
                               a.dtype, stream);
    if (st != TTCD_OK) return st;
    ttcd::MergeArgs m = {a.o_s, nullptr, a.o_s, nullptr, a.o_t, a.B, n0, a.Hq, a.D, n0,
                         a.os[0], a.os[1], a.os[2], a.os[0], a.os[1], a.os[2]};
    st = from_hip(ttcd::launch_lse_merge(m, et, hs), "lse variant copy launch");
    if (st != TTCD_OK) return st;
  }
  for (int64_t r0 = n0; r0 < a.Tq; r0 += rows) {
    const int r1 = (int)(r0 + rows < a.Tq ? r0 + rows : a.Tq);
    const int tc = r1 - (int)r0, tk = qoff + r1;
    char* o_f = ws;
    float* lse_s = reinterpret_cast<float*>(ws + align_up((size_t)a.B * tc * a.Hq * a.D * es));
    float* lse_f = reinterpret_cast<float*>(reinterpret_cast<char*>(lse_s) +
                                            align_up((size_t)a.B * a.Hq * tc * 4));
    const int64_t fs[4] = {(int64_t)tc * a.Hq * a.D, (int64_t)a.Hq * a.D, a.D, 1};
    const void* qc = q + (size_t)r0 * a.qs[1] * es;
    void* osc = o_s + (size_t)r0 * a.os[1] * es;
    st = ttcd_band_attn_kv_fwd(qc, a.k, a.v, osc, lse_s, a.B, tc, tk, a.Hq, a.Hkv, a.D, a.qs,
                               a.ks, a.vs, a.os, 0, a.WS, a.sm_scale, a.rescale_log2, a.dtype,
                               stream);
    if (st != TTCD_OK) return st;
    st = ttcd_band_attn_kv_fwd(qc, a.k, a.v, o_f, lse_f, a.B, tc, tk, a.Hq, a.Hkv, a.D, a.qs,
                               a.ks, a.vs, fs, a.WS, a.WT, a.sm_scale, a.rescale_log2, a.dtype,
                               stream);
    if (st != TTCD_OK) return st;
    ttcd::MergeArgs m = {osc, lse_s, o_f, lse_f, o_t + (size_t)r0 * a.os[1] * es, a.B, tc, a.Hq,
                         a.D, 0, a.os[0], a.os[1], a.os[2], fs[0], fs[1], fs[2]};
    st = from_hip(ttcd::launch_lse_merge(m, et, hs), "lse variant merge launch");
    if (st != TTCD_OK) return st;
  }
  return ok();
}

}  // namespace

size_t ttcd_lse_dual_window_attn_workspace_bytes(int B, int Tq, int Tk, int Hq, int D,
                                                 int window_s) {
  if (B < 1 || Tq < 1 || Tq > Tk || Hq < 1 || D < 1 || window_s < 1) return 0;
  LseDual a = {};
  a.B = B;
  a.Tq = Tq;
  a.Tk = Tk;
  a.Hq = Hq;
  a.D = D;
  a.WS = window_s;
  const int64_t need = Tq - a.n0();
  return need > 0 ? a.chunk_bytes(need) : 0;
}

ttcd_status ttcd_lse_dual_window_attn_fwd(const void* q, const void* k, const void* v,
                                          void* o_t, void* o_s, int B, int Tq, int Tk, int Hq,
                                          int Hkv, int D, const int64_t q_stride[4],
                                          const int64_t k_stride[4], const int64_t v_stride[4],
                                          const int64_t o_stride[4], int window_t, int window_s,
                                          float sm_scale, float rescale_log2, ttcd_dtype dtype,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  LseDual a = {q, k, v, o_t, o_s, B, Tq, Tk, Hq, Hkv, D, 0, 0, q_stride, k_stride, v_stride,
               o_stride, sm_scale, rescale_log2, dtype};
  ttcd_status st = check_lse_dual(&a, window_t, window_s);
  if (st != TTCD_OK) return st;
  if (workspace_bytes > 0 && (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255u)))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "workspace must be non-null and 256-byte aligned");
  return run_lse_dual(a, static_cast<char*>(workspace), workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free LSE variant. Its scratch is a file-scope device array: one
// copy per GPU the library runs on, held until the process ends. On the host
// the array's name is only a stand-in, never a device address: the address
// is resolved once per device with hipGetSymbolAddress (that device current)
// and only that pointer is passed to kernels. Every call on one GPU shares the
// array; the variant writes each scratch element before reading it, so
// nothing needs clearing, but calls that overlap in time on one GPU (different
// streams without ordering) race on it.
namespace {
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
}  // namespace
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device of `stream` (the current device
// for the null stream), resolved on first use there.
ttcd_status scratch_for(void* stream, char** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return from_hip(e, "hipGetDevice");
  int dev = cur;
  if (stream != nullptr) {
    hipDevice_t d = 0;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &d);
    if (e != hipSuccess) return from_hip(e, "hipStreamGetDevice");
    dev = d;
  }
  if (dev < 0 || dev >= kMaxDevices)
    return fail(TTCD_ERR_UNSUPPORTED, "device %d beyond the %d the scratch table holds", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur) {
      e = hipSetDevice(dev);
      if (e != hipSuccess) return from_hip(e, "hipSetDevice");
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess && e2 != hipSuccess) e = e2;
    }
    if (e != hipSuccess) return from_hip(e, "hipGetSymbolAddress(scratch)");
    if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & 255u) != 0)
      return fail(TTCD_ERR_HIP, "scratch symbol has no 256-byte aligned device address");
    g_scratch_ptr[dev] = p;
  }
  *out = static_cast<char*>(g_scratch_ptr[dev]);
  return TTCD_OK;
}
}  // namespace

size_t ttcd_lse_dual_window_attn_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

ttcd_status ttcd_lse_dual_window_attn_noalloc_fwd(
    const void* q, const void* k, const void* v, void* o_t, void* o_s, int B, int Tq, int Tk,
    int Hq, int Hkv, int D, const int64_t q_stride[4], const int64_t k_stride[4],
    const int64_t v_stride[4], const int64_t o_stride[4], int window_t, int window_s,
    float sm_scale, float rescale_log2, ttcd_dtype dtype, void* stream) {
  LseDual a = {q, k, v, o_t, o_s, B, Tq, Tk, Hq, Hkv, D, 0, 0, q_stride, k_stride, v_stride,
               o_stride, sm_scale, rescale_log2, dtype};
  ttcd_status st = check_lse_dual(&a, window_t, window_s);
  if (st != TTCD_OK) return st;
  if (a.n0() < a.Tq && a.rows_fitting(kNoAllocScratchBytes) < 1)
    return fail(TTCD_ERR_UNSUPPORTED,
                "B * Hq too large for the %zu-byte scratch: one query row needs %zu bytes",
                kNoAllocScratchBytes, a.chunk_bytes(1));
  char* ws = nullptr;
  st = scratch_for(stream, &ws);
  if (st != TTCD_OK) return st;
  return run_lse_dual(a, ws, kNoAllocScratchBytes, stream);
}

ttcd_status ttcd_causal_dwconv_chunked_fwd(const void* x, const void* w, void* y, int64_t N,
                                           int C, int D, int K, ttcd_dtype x_dtype,
                                           ttcd_dtype w_dtype, void* stream) {
  if (!x || !w || !y) return fail(TTCD_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (N < 0 || C < 0 || D < 0) return fail(TTCD_ERR_INVALID_ARGUMENT, "negative extent");
  if (K < 1 || K > 64) return fail(TTCD_ERR_INVALID_ARGUMENT, "kernel size %d not in [1, 64]", K);
  if ((unsigned)x_dtype > TTCD_DTYPE_F32 || (unsigned)w_dtype > TTCD_DTYPE_F32)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "unknown dtype");
  if (N == 0 || C == 0 || D == 0) return ok();
  return from_hip(ttcd::launch_dwconv(x, w, y, N, C, D, K, elem(x_dtype), elem(w_dtype),
                                      static_cast<hipStream_t>(stream)),
                  "depthwise conv launch");
}

ttcd_status ttcd_rope_table_fwd(void* cos_table, void* sin_table, const float* inv_freq,
                                int rows, int half_dim, ttcd_dtype dtype, void* stream) {
  if (!cos_table || !sin_table || !inv_freq)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (rows < 0 || half_dim < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "need rows >= 0 and half_dim >= 1 (got %d, %d)", rows,
                half_dim);
  if (dtype != TTCD_DTYPE_BF16 && dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "table dtype must be bf16 or f16");
  if (rows == 0) return ok();
  return from_hip(ttcd::launch_rope_table(cos_table, sin_table, inv_freq, rows, half_dim,
                                          elem(dtype), static_cast<hipStream_t>(stream)),
                  "rope table launch");
}

ttcd_status ttcd_qk_norm_rope_fwd(const void* q, const void* k, void* q_out, void* k_out,
                                  const void* q_norm_w, const void* k_norm_w, ttcd_dtype w_dtype,
                                  float eps, const void* cos_table, const void* sin_table,
                                  int table_rows, int B, int T, int Hq, int Hkv, int D,
                                  const int64_t q_stride[4], const int64_t k_stride[4],
                                  const int64_t q_out_stride[4], const int64_t k_out_stride[4],
                                  int seqlen_offset, ttcd_dtype dtype, void* stream) {
  if (!q || !k || !q_out || !k_out || !cos_table || !sin_table)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "null tensor pointer");
  if (!q_stride || !k_stride || !q_out_stride || !k_out_stride)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "null stride array");
  if ((q_norm_w == nullptr) != (k_norm_w == nullptr))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "give both norm weights or neither");
  if (B < 1 || T < 1 || Hq < 1 || Hkv < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "B, T, Hq, Hkv must be >= 1 (got %d, %d, %d, %d)", B,
                T, Hq, Hkv);
  if (D != 64 && D != 128)
    return fail(TTCD_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", D);
  if (dtype != TTCD_DTYPE_BF16 && dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "q/k dtype must be bf16 or f16");
  if (q_norm_w && (unsigned)w_dtype > TTCD_DTYPE_F32)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "unknown norm weight dtype");
  if (!(eps >= 0.f) || !isfinite(eps))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
  if (seqlen_offset < 0) return fail(TTCD_ERR_INVALID_ARGUMENT, "seqlen_offset must be >= 0");
  if ((int64_t)seqlen_offset + T > (int64_t)table_rows)
    return fail(TTCD_ERR_INVALID_ARGUMENT,
                "rotary tables too short: seqlen_offset + T = %lld > table rows %d",
                (long long)seqlen_offset + T, table_rows);
  const int64_t* all[4] = {q_stride, k_stride, q_out_stride, k_out_stride};
  for (int t = 0; t < 4; ++t) {
    if (all[t][3] != 1)
      return fail(TTCD_ERR_INVALID_ARGUMENT, "head_dim must be contiguous (d-stride 1)");
    for (int i = 0; i < 3; ++i)
      if (all[t][i] % 8 != 0 || all[t][i] < 0)
        return fail(TTCD_ERR_UNSUPPORTED,
                    "strides must be non-negative multiples of 8 elements (16-byte rows)");
  }
  if (!aligned16(q) || !aligned16(k) || !aligned16(q_out) || !aligned16(k_out) ||
      !aligned16(cos_table) || !aligned16(sin_table))
    return fail(TTCD_ERR_UNSUPPORTED, "tensor base pointers must be 16-byte aligned");
  ttcd::PrologueArgs a = {};
  a.q = q;
  a.k = k;
  a.q_out = q_out;
  a.k_out = k_out;
  a.q_w = q_norm_w;
  a.k_w = k_norm_w;
  a.cos = cos_table;
  a.sin = sin_table;
  a.eps = eps;
  a.offset = seqlen_offset;
  a.B = B;
  a.T = T;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.D = D;
  a.q_sb = q_stride[0];
  a.q_st = q_stride[1];
  a.q_sh = q_stride[2];
  a.k_sb = k_stride[0];
  a.k_st = k_stride[1];
  a.k_sh = k_stride[2];
  a.qo_sb = q_out_stride[0];
  a.qo_st = q_out_stride[1];
  a.qo_sh = q_out_stride[2];
  a.ko_sb = k_out_stride[0];
  a.ko_st = k_out_stride[1];
  a.ko_sh = k_out_stride[2];
  return from_hip(ttcd::launch_qk_norm_rope(a, elem(dtype), elem(w_dtype),
                                            static_cast<hipStream_t>(stream)),
                  "qk norm + rope launch");
}

ttcd_status ttcd_dual_residual_rmsnorm_fwd(const void* attn_t, const void* attn_s,
                                           const void* residual, const void* norm_w,
                                           ttcd_dtype w_dtype, float eps, void* hidden_out,
                                           void* residual_out, void* student_out,
                                           int64_t rows, int hidden, ttcd_dtype dtype,
                                           void* stream) {
  if (!attn_t || !attn_s || !residual || !norm_w || !hidden_out || !residual_out ||
      !student_out)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (rows < 0 || hidden < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "need rows >= 0 and hidden >= 1");
  if (hidden % 8 != 0 || hidden > 2048)
    return fail(TTCD_ERR_UNSUPPORTED, "hidden size %d not supported (a multiple of 8, <= 2048)",
                hidden);
  if (dtype != TTCD_DTYPE_BF16 && dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "activation dtype must be bf16 or f16");
  if ((unsigned)w_dtype > TTCD_DTYPE_F32)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "unknown norm weight dtype");
  if (!(eps >= 0.f) || !isfinite(eps))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
  const void* all[6] = {attn_t, attn_s, residual, hidden_out, residual_out, student_out};
  for (int i = 0; i < 6; ++i)
    if (!aligned16(all[i]))
      return fail(TTCD_ERR_UNSUPPORTED, "tensor base pointers must be 16-byte aligned");
  if (w_dtype != TTCD_DTYPE_F32 && !aligned16(norm_w))
    return fail(TTCD_ERR_UNSUPPORTED, "16-bit norm weights must be 16-byte aligned");
  if (rows == 0) return ok();
  return from_hip(ttcd::launch_dual_residual_rmsnorm(
                      attn_t, attn_s, residual, norm_w, elem(w_dtype), eps, hidden_out,
                      residual_out, student_out, rows, hidden, elem(dtype),
                      static_cast<hipStream_t>(stream)),
                  "dual residual rmsnorm launch");
}

ttcd_status ttcd_rmsnorm_fwd(const void* x, const void* residual, const void* norm_w,
                             ttcd_dtype w_dtype, float eps, void* y, void* residual_out,
                             int64_t rows, int hidden, ttcd_dtype dtype, void* stream) {
  if (!x || !norm_w || !y) return fail(TTCD_ERR_INVALID_ARGUMENT, "null pointer argument");
  if ((residual == nullptr) != (residual_out == nullptr))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "pass residual and residual_out both or neither");
  if (rows < 0 || hidden < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "need rows >= 0 and hidden >= 1");
  if (hidden % 8 != 0 || hidden > 2048)
    return fail(TTCD_ERR_UNSUPPORTED, "hidden size %d not supported (a multiple of 8, <= 2048)",
                hidden);
  if (dtype != TTCD_DTYPE_BF16 && dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "activation dtype must be bf16 or f16");
  if ((unsigned)w_dtype > TTCD_DTYPE_F32)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "unknown norm weight dtype");
  if (!(eps >= 0.f) || !isfinite(eps))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
  const void* all[4] = {x, y, residual, residual_out};
  for (int i = 0; i < 4; ++i)
    if (all[i] && !aligned16(all[i]))
      return fail(TTCD_ERR_UNSUPPORTED, "tensor base pointers must be 16-byte aligned");
  if (w_dtype != TTCD_DTYPE_F32 && !aligned16(norm_w))
    return fail(TTCD_ERR_UNSUPPORTED, "16-bit norm weights must be 16-byte aligned");
  if (rows == 0) return ok();
  return from_hip(ttcd::launch_dual_residual_rmsnorm(
                      x, nullptr, residual, norm_w, elem(w_dtype), eps, y, residual_out, nullptr,
                      rows, hidden, elem(dtype), static_cast<hipStream_t>(stream)),
                  "rmsnorm launch");
}

ttcd_status ttcd_add_rmsnorm_fwd(const void* x, const void* residual, const void* norm_w,
                                 ttcd_dtype w_dtype, float eps, void* y, void* sum_out,
                                 int64_t rows, int hidden, ttcd_dtype dtype, void* stream) {
  if (!x || !residual || !norm_w || !y || !sum_out)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (rows < 0 || hidden < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "need rows >= 0 and hidden >= 1");
  if (hidden % 8 != 0 || hidden > 2048)
    return fail(TTCD_ERR_UNSUPPORTED, "hidden size %d not supported (a multiple of 8, <= 2048)",
                hidden);
  if (dtype != TTCD_DTYPE_BF16 && dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "activation dtype must be bf16 or f16");
  if ((unsigned)w_dtype > TTCD_DTYPE_F32)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "unknown norm weight dtype");
  if (!(eps >= 0.f) || !isfinite(eps))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
  const void* all[4] = {x, residual, y, sum_out};
  for (int i = 0; i < 4; ++i)
    if (!aligned16(all[i]))
      return fail(TTCD_ERR_UNSUPPORTED, "tensor base pointers must be 16-byte aligned");
  if (w_dtype != TTCD_DTYPE_F32 && !aligned16(norm_w))
    return fail(TTCD_ERR_UNSUPPORTED, "16-bit norm weights must be 16-byte aligned");
  if (rows == 0) return ok();
  return from_hip(ttcd::launch_dual_residual_rmsnorm(
                      x, nullptr, residual, norm_w, elem(w_dtype), eps, y, sum_out, nullptr,
                      rows, hidden, elem(dtype), static_cast<hipStream_t>(stream), true),
                  "add rmsnorm launch");
}

ttcd_status ttcd_swiglu_fwd(const void* gate, const void* up, void* out, int64_t rows, int cols,
                            int64_t gate_stride, int64_t up_stride, int64_t out_stride,
                            ttcd_dtype dtype, void* stream) {
  if (!gate || !up || !out) return fail(TTCD_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (rows < 0 || cols < 1) return fail(TTCD_ERR_INVALID_ARGUMENT, "need rows >= 0, cols >= 1");
  if (gate_stride < cols || up_stride < cols || out_stride < cols)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "row strides must be >= cols");
  if (dtype != TTCD_DTYPE_BF16 && dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "dtype must be bf16 or f16");
  if (cols % 8 != 0 || gate_stride % 8 != 0 || up_stride % 8 != 0 || out_stride % 8 != 0)
    return fail(TTCD_ERR_UNSUPPORTED, "cols and row strides must be multiples of 8");
  if (!aligned16(gate) || !aligned16(up) || !aligned16(out))
    return fail(TTCD_ERR_UNSUPPORTED, "tensor base pointers must be 16-byte aligned");
  if (rows == 0) return ok();
  return from_hip(ttcd::launch_swiglu(gate, up, out, rows, cols, gate_stride, up_stride,
                                      out_stride, elem(dtype), static_cast<hipStream_t>(stream)),
                  "swiglu launch");
}

ttcd_status ttcd_ttt_features_fwd(const void* gu_t, const void* gu_s, int64_t gu_stride,
                                  const void* conv_t, const void* conv_s, ttcd_dtype w_dtype,
                                  int kernel_size, void* z, void* z_hat, void* diff, int B,
                                  int nchunk, int chunk, int inter, ttcd_dtype dtype,
                                  void* stream) {
  if (!gu_t || !gu_s || !z || !z_hat || (nchunk > 1 && !diff))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (B < 1 || nchunk < 1 || chunk < 1 || inter < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "need B, nchunk, chunk, inter >= 1");
  if (gu_stride < 2 * (int64_t)inter)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "gate|up row stride must be >= 2 * inter");
  if (kernel_size < 1 || ((conv_t || conv_s) && kernel_size > 8))
    return fail(TTCD_ERR_UNSUPPORTED, "conv kernel size must be in 1..8");
  if (dtype != TTCD_DTYPE_BF16 && dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "dtype must be bf16 or f16");
  if ((unsigned)w_dtype > TTCD_DTYPE_F32)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "unknown conv weight dtype");
  if (inter % 8 != 0 || gu_stride % 8 != 0)
    return fail(TTCD_ERR_UNSUPPORTED, "inter and the gate|up row stride must be multiples of 8");
  const void* all[5] = {gu_t, gu_s, z, z_hat, diff};
  for (int i = 0; i < 5; ++i)
    if (all[i] && !aligned16(all[i]))
      return fail(TTCD_ERR_UNSUPPORTED, "tensor base pointers must be 16-byte aligned");
  ttcd::TttFeatureArgs a{gu_t, gu_s, gu_stride, conv_t, conv_s, (conv_t || conv_s) ? kernel_size : 1,
                         z, z_hat, diff, B, nchunk, chunk, inter};
  return from_hip(ttcd::launch_ttt_features(a, elem(dtype), elem(w_dtype),
                                            static_cast<hipStream_t>(stream)),
                  "ttt features launch");
}

ttcd_status ttcd_ttt_proj_beta_t_fwd(const void* pd, int64_t pd_stride, const void* beta,
                                    int64_t beta_batch_stride, void* pdt, int B, int nupd,
                                    int chunk, int H, ttcd_dtype dtype, void* stream) {
  if (!pd || !pdt) return fail(TTCD_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (B < 1 || nupd < 1 || chunk < 1 || H < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "need B, nupd, chunk, H >= 1");
  if (pd_stride < H || (beta && beta_batch_stride < (int64_t)nupd * chunk))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "pd row stride must be >= H and the beta batch "
                                           "stride >= nupd * chunk");
  if (dtype != TTCD_DTYPE_BF16 && dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "dtype must be bf16 or f16");
  if ((int64_t)B * nupd > 65535)
    return fail(TTCD_ERR_UNSUPPORTED, "B * nupd above 65535 (grid z)");
  ttcd::TttProjBetaArgs a{pd, pd_stride, beta, beta_batch_stride, pdt, B, nupd, chunk, H};
  return from_hip(ttcd::launch_ttt_proj_beta_t(a, elem(dtype), static_cast<hipStream_t>(stream)),
                  "ttt pd*beta launch");
}

ttcd_status ttcd_ttt_scan_fwd(const void* dw, const void* w_cur, float lr, void* steps_t,
                              void* w_next, int nupd, int nsteps, int H, int inter,
                              ttcd_dtype dtype, void* stream) {
  if (!w_cur || !steps_t || (nupd > 0 && !dw))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (H < 1 || inter < 1 || nupd < 0 || nsteps < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "need H, inter, nsteps >= 1 and nupd >= 0");
  // chunk s of the group uses cs[s - 1]: there must be one for every step but the first
  if (nsteps > nupd + 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "nsteps (%d) must be <= nupd + 1 (%d)", nsteps,
                nupd + 1);
  if (w_next && nupd < 1)
    return fail(TTCD_ERR_INVALID_ARGUMENT, "w_next needs at least one update");
  if (!isfinite(lr)) return fail(TTCD_ERR_INVALID_ARGUMENT, "lr must be finite");
  if (dtype != TTCD_DTYPE_BF16 && dtype != TTCD_DTYPE_F16)
    return fail(TTCD_ERR_UNSUPPORTED, "dtype must be bf16 or f16");
  ttcd::TttScanArgs a{dw, w_cur, lr, steps_t, w_next, nupd, nsteps, H, inter};
  return from_hip(ttcd::launch_ttt_scan(a, elem(dtype), static_cast<hipStream_t>(stream)),
                  "ttt scan launch");
}

ttcd_status ttcd_attn_schedule_coverage(int T, int dual, int window_s, int window_t,
                                        int gqa_group, int32_t* counts_near,
                                        int32_t* counts_far) {
  using namespace ttcd;
  if (T < 1 || gqa_group < 1 || !counts_near || (dual && !counts_far))
    return fail(TTCD_ERR_INVALID_ARGUMENT, "bad coverage arguments");
  Schedule sc;
  if (dual) {
    if (window_t < 0) window_t = T;
    if (window_s < 1 || window_s > window_t)
      return fail(TTCD_ERR_INVALID_ARGUMENT, "need 1 <= window_s <= window_t");
    sc = make_dual_schedule(T, window_s, window_t, wave_rows(gqa_group));
  } else {
    if (window_s < 0 || window_t <= window_s)
      return fail(TTCD_ERR_INVALID_ARGUMENT, "need 0 <= band_lo < band_hi");
    sc = make_band_schedule(T, window_s, window_t, wave_rows(gqa_group));
  }
  // Workgroup geometry as launched (attn.hip): 4 waves over 4R consecutive
  // tokens, wave w owning rows r0 = t0 + R*w (R = 16 for an even gqa_group,
  // else 32).
  const int R = sc.rows;
  const int span = wg_span_tokens(gqa_group);
  const int nwg = (T + span - 1) / span;
  for (int qb = 0; qb < nwg; ++qb) {
    const int t0 = qb * span;
    const int t_last = (t0 + span < T ? t0 + span : T) - 1;
    int n_hi, n_lo;
    if (!sc.wg_range(t0, t_last, &n_hi, &n_lo)) continue;
    auto r0_of_wave = [&](int wv) { return t0 + wv * R; };
    const SlotPlan sp = make_slot_plan(sc, r0_of_wave, n_hi, n_lo);
    const int nslot = sp.slots();
    for (int w = 0; w < kWaves; ++w) {
      const int r0 = t0 + w * R;
      if (r0 >= T) continue;
      bool student_done = false;
      const WaveSlots ws(sc, r0);  // the kernel's closed form
      // past the last slot the kernel's words load and fold nothing
      for (int k = nslot; k < nslot + 2; ++k)
        if (slot_word(sc, sp, ws, nslot, true, T, k) != 0)
          return fail(TTCD_ERR_UNSUPPORTED, "schedule error: word of slot %d past the end", k);
      for (int k = 0; k < nslot; ++k) {
        bool repeat;
        const int n = sp.tile(k, &repeat);
        const int j0 = sc.tile_start(n);
        const int act = slot_action(sc, r0, j0, repeat);
        if (ws.act(n, repeat) != act)
          return fail(TTCD_ERR_UNSUPPORTED, "schedule error: closed-form action %d != %d (r0=%d n=%d)",
                      ws.act(n, repeat), act, r0, n);
        // The kernel reads the slot only through its word: decode it and
        // check every field against the plan and the per-tile predicates.
        const uint32_t wd = slot_word(sc, sp, ws, nslot, true, T, k);
        const bool interior = j0 >= 0 && j0 + kBlockN <= T;
        if (n < 0 || word_tile(wd) != n || word_j0(sc, wd) != j0 || !(wd & kWordLoad) ||
            ((wd & kWordInterior) != 0) != interior)
          return fail(TTCD_ERR_UNSUPPORTED, "schedule error: slot word tile/load (r0=%d k=%d)", r0, k);
        if (slot_word(sc, sp, ws, nslot, false, T, k) != (wd & ~63u) + (wd & (kWordLoad | kWordInterior)))
          return fail(TTCD_ERR_UNSUPPORTED, "schedule error: idle-wave word (r0=%d k=%d)", r0, k);
        const bool w_active = (wd & kWordActive) != 0;
        if (w_active != (act != kSkip) ||
            ((wd & kWordFar) != 0) != (act == kBand2 || act == kFar) ||
            ((wd & kWordLast) != 0) != (act == kStudentLast))
          return fail(TTCD_ERR_UNSUPPORTED, "schedule error: slot word action (r0=%d k=%d)", r0, k);
        if (act != kSkip) {
          const Band b = (act == kBand2 || act == kFar) ? sc.p2 : sc.p1;
          const Band wb = word_band(sc, wd);
          if (wb.lo != b.lo || wb.hi != b.hi)
            return fail(TTCD_ERR_UNSUPPORTED, "schedule error: slot word band (r0=%d n=%d)", r0, n);
          const bool need_mask = !wave_full(r0, R, b, j0);
          if (ws.mask(n, act) != need_mask || ((wd & kWordMask) != 0) != need_mask)
            return fail(TTCD_ERR_UNSUPPORTED, "schedule error: closed-form mask (r0=%d n=%d)", r0, n);
        } else if (wd & kWordMask) {
          return fail(TTCD_ERR_UNSUPPORTED, "schedule error: mask on a skipped slot (r0=%d n=%d)", r0, n);
        }
        // From here on the replay folds what the word says, as the kernel does.
        if (!w_active) continue;
        const bool far = (wd & kWordFar) != 0;
        if (sc.dual && !far && student_done)
          return fail(TTCD_ERR_UNSUPPORTED, "schedule error: student keys after emit (r0=%d k=%d)",
                      r0, k);
        if (sc.dual && far && !student_done)
          return fail(TTCD_ERR_UNSUPPORTED, "schedule error: far keys before emit (r0=%d k=%d)",
                      r0, k);
        const Band band = word_band(sc, wd);
        const bool full = (wd & kWordMask) == 0;
        const int wj0 = word_j0(sc, wd);
        for (int i = r0; i < r0 + R && i < T; ++i) {
          for (int j = wj0; j < wj0 + kBlockN; ++j) {
            if (!(full || visible(i, j, band, T))) continue;
            if (j < 0 || j >= T)
              return fail(TTCD_ERR_UNSUPPORTED, "schedule error: key %d out of range", j);
            int32_t* cnt = far ? counts_far : counts_near;
            cnt[(int64_t)i * T + j] += 1;
          }
        }
        if (wd & kWordLast) student_done = true;
      }
      if (sc.dual && !student_done && sc.p1.lo < sc.p1.hi)
        return fail(TTCD_ERR_UNSUPPORTED, "schedule error: student output never written (r0=%d)",
                    r0);
    }
  }
  return ok();
}

}  // extern "C"
