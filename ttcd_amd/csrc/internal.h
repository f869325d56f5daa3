// internal.h - launcher interface between the C ABI (api.hip) and the
// gfx950 kernels (attn.hip, conv.hip, merge.hip, prologue.hip, epilogue.hip).
// Not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "schedule.h"

namespace ttcd {

enum class Elem { BF16 = 0, F16 = 1, F32 = 2 };

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o_t;      // final output (teacher for the dual kernel, band output otherwise)
  void* o_s;      // student output (dual kernel only)
  float* lse_t;   // optional (B, Hq, Tq)
  float* lse_s;   // optional (B, Hq, Tq), dual kernel only
  int64_t q_sb, q_st, q_sh;
  int64_t k_sb, k_st, k_sh;
  int64_t v_sb, v_st, v_sh;
  int64_t o_sb, o_st, o_sh;
  int B, T, Hq, Hkv, G;  // T: keys (Tk); query rows are absolute positions q_off..T-1
  int q_off;      // Tk - Tq: absolute position of query row 0 (flash-attention's
                  // bottom-right alignment; 0 when Tq == Tk)
  int qb0;        // first query tile launched: q_off / (4 * sched.rows)
  int nqb;        // query tiles of 4 * sched.rows tokens per (b, head group) launched
  int nwg;        // workgroups launched (set by the launcher)
  float c;        // sm_scale * log2(e)
  float rescale_log2;  // lazy online softmax: the reference max moves when a row max
                       // exceeds it by more than 2^rescale_log2 (0: exact running max)
  Schedule sched;
  int64_t lse_sb, lse_sh;  // LSE strides per batch entry / head (rows are contiguous)
  // Packed sequences (null for fixed-length batches): sequence b is rows
  // cu_seqlens[b] .. cu_seqlens[b+1]-1 of every tensor (B sequences, `total`
  // rows); its schedule is built in the kernel from T = its length and the
  // windows below (dual: win_a = w_S, win_b = w_T; band: lo, hi).
  const int* cu_seqlens;
  int total;
  int win_a, win_b;
};

// Default lazy-rescale threshold (log2 units) of the attention entry points
// that take none.
constexpr float kDefaultRescaleLog2 = 8.0f;

// Launch the dual-window (sched.dual == 1) or single-band kernel.
hipError_t launch_attn(const AttnArgs& a, int D, Elem dtype, hipStream_t stream);

struct PrologueArgs {
  const void* q;
  const void* k;
  void* q_out;
  void* k_out;
  const void* q_w;    // RMSNorm weights (both null: no norm)
  const void* k_w;
  const void* cos;    // (table_rows, D/2) contiguous, input dtype
  const void* sin;
  float eps;
  int offset;         // position of token 0 in the tables
  int B, T, Hq, Hkv, D;
  int64_t q_sb, q_st, q_sh;
  int64_t k_sb, k_st, k_sh;
  int64_t qo_sb, qo_st, qo_sh;
  int64_t ko_sb, ko_st, ko_sh;
};

// Fused q/k RMSNorm + rotary embedding (prologue.hip).
hipError_t launch_qk_norm_rope(const PrologueArgs& a, Elem dtype, Elem wt, hipStream_t stream);

// cos/sin tables: row t, column i = cos/sin(fp32(t) * inv_freq[i]) rounded to dtype.
hipError_t launch_rope_table(void* cos_t, void* sin_t, const float* inv_freq, int rows, int half,
                             Elem dtype, hipStream_t stream);

// Teacher and student residual add + RMSNorm of the attention outputs (epilogue.hip).
hipError_t launch_dual_residual_rmsnorm(const void* a_t, const void* a_s, const void* res,
                                        const void* w, Elem wt, float eps, void* y_t,
                                        void* res_out, void* y_s, int64_t rows, int H,
                                        Elem dtype, hipStream_t stream, bool round_sum = false);

// TTT MLP feature pass (ttt.hip). Rows are b-major, then chunk, then position.
struct TttFeatureArgs {
  const void* gu_t;  // teacher (rows, 2*I) gate | up, row stride gu_st
  const void* gu_s;  // student, same layout
  int64_t gu_st;
  const void* w_t;   // teacher conv weight (I, K) or null
  const void* w_s;   // student conv weight (I, K) or null
  int K;
  void* z;           // (rows, I) teacher features
  void* z_hat;       // (rows, I) student features after the student conv
  void* diff;        // (B * (nchunk - 1) * C, I)
  int B, nchunk, C, I;
};

hipError_t launch_swiglu(const void* gate, const void* up, void* out, int64_t rows, int cols,
                         int64_t gate_stride, int64_t up_stride, int64_t out_stride, Elem dtype,
                         hipStream_t stream);
hipError_t launch_ttt_features(const TttFeatureArgs& a, Elem dtype, Elem w_dtype,
                               hipStream_t stream);

// The TTT update scan (ttt.hip).
struct TttProjBetaArgs {
  const void* pd;      // (B * nupd * C, H) rows, row stride pd_stride
  int64_t pd_stride;
  const void* beta;    // per token: b * beta_sb + c * C + t, or null (no scaling)
  int64_t beta_sb;
  void* pdt;           // (B * nupd, H, C) contiguous
  int B, nupd, C, H;
};
struct TttScanArgs {
  const void* dw;      // (nupd, H, I) contiguous
  const void* w_cur;   // (H, I) contiguous
  float lr;            // the learning rate as stored in the dtype
  void* steps_t;       // (nsteps, I, H) contiguous: W_step transposed
  void* w_next;        // (H, I) or null: W_cur + cs[nupd - 1]
  int nupd, nsteps, H, I;
};
hipError_t launch_ttt_proj_beta_t(const TttProjBetaArgs& a, Elem dtype, hipStream_t stream);
hipError_t launch_ttt_scan(const TttScanArgs& a, Elem dtype, hipStream_t stream);

hipError_t launch_dwconv(const void* x, const void* w, void* y, int64_t N, int C,
                         int D, int K, Elem xt, Elem wt, hipStream_t stream);

// Log-sum-exp merge of two partials (merge.hip). Rows t < row_start copy o_s.
struct MergeArgs {
  const void* o_s;      // (B, T, H, D), strides sb / st / sh (o_t shares them)
  const float* lse_s;   // (B, H, T) contiguous
  const void* o_f;      // (B, T, H, D), strides f_sb / f_st / f_sh
  const float* lse_f;   // (B, H, T) contiguous
  void* o_t;
  int B, T, H, D, row_start;
  int64_t sb, st, sh;
  int64_t f_sb, f_st, f_sh;
};
hipError_t launch_lse_merge(const MergeArgs& a, Elem dtype, hipStream_t stream);

}  // namespace ttcd
