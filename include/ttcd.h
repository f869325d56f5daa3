/*
 * ttcd.h - plain C ABI of the MI355X (gfx950) dual-window attention and
 * chunked causal depthwise conv library (libttcd_amd.so).
 *
 * Every buffer is a device pointer owned by the caller; the library never
 * allocates or frees memory. Strides are in elements; the last (head_dim /
 * channel) dimension must be contiguous. All kernels are launched on the
 * caller's stream (`stream` is a hipStream_t passed as void*, NULL = the
 * legacy default stream) and return without synchronising. Functions are
 * reentrant and thread-safe; the only global state is a thread-local error
 * message (ttcd_last_error).
 *
 * Windows follow flash-attention's window_size=(W-1, 0): key j is visible to
 * query i iff 0 <= i - j <= W - 1. Softmax is computed in fp32; LSE outputs
 * are natural-log, fp32, laid out (B, H, T) contiguous.
 */
#ifndef TTCD_H_
#define TTCD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TTCD_ABI_VERSION 2

typedef enum ttcd_status {
  TTCD_OK = 0,
  TTCD_ERR_INVALID_ARGUMENT = 1, /* bad shape, window, stride, null pointer */
  TTCD_ERR_UNSUPPORTED = 2,      /* valid request this build does not cover */
  TTCD_ERR_HIP = 3               /* the HIP runtime reported a launch error */
} ttcd_status;

typedef enum ttcd_dtype {
  TTCD_DTYPE_BF16 = 0,
  TTCD_DTYPE_F16 = 1,
  TTCD_DTYPE_F32 = 2
} ttcd_dtype;

/* Human-readable name of a status code. */
const char* ttcd_status_string(ttcd_status status);

/* Message describing the last error returned on the calling thread. */
const char* ttcd_last_error(void);

/* TTCD_ABI_VERSION of the loaded library. */
int ttcd_abi_version(void);

/*
 * One-pass dual-window causal GQA attention (forward, prefill, Tq == Tk;
 * ttcd_dual_window_attn_kv_fwd below takes Tq <= Tk).
 * Replaces fused_dual_window_attn / _fused_dual_swa_fwd
 * (profiling/fused_dual_attn.py:244-272, kernel :44-241).
 *
 * q: (B, T, Hq, D); k, v: (B, T, Hkv, D); o_t, o_s: (B, T, Hq, D), all of
 * `dtype` (BF16 or F16), D in {64, 128}, Hq % Hkv == 0, head h reads kv head
 * h / (Hq / Hkv). *_stride[4] = element strides of (b, t, h, d); d-stride 1,
 * the others non-negative multiples of 8; the k and v token strides at most
 * 2^25 (TTCD_ERR_UNSUPPORTED above). These stride rules hold for every
 * attention entry point below.
 * o_t and o_s share o_stride. window_t >= T (or < 0) means full causal.
 * Requires 1 <= window_s <= window_t. lse_t / lse_s may be NULL; when given
 * they receive log(sum_j exp(sm_scale * q.k_j)) over each window, (B, Hq, T).
 */
ttcd_status ttcd_dual_window_attn_fwd(
    const void* q, const void* k, const void* v, void* o_t, void* o_s,
    float* lse_t, float* lse_s, int B, int T, int Hq, int Hkv, int D,
    const int64_t q_stride[4], const int64_t k_stride[4],
    const int64_t v_stride[4], const int64_t o_stride[4], int window_t,
    int window_s, float sm_scale, ttcd_dtype dtype, void* stream);

/*
 * Single-band causal GQA attention over keys with band_lo <= i - j < band_hi.
 * band_lo = 0, band_hi = W is the flash-attention windowed call
 * (flash_attn_func(..., causal=True, window_size=(W-1, 0)) as called at
 * profiling/lse_dual_attn.py:22-23); band_lo = WS, band_hi = WT is the far
 * band of the LSE-combination variant, computed on the unshifted tensors
 * (replaces the shifted call at profiling/lse_dual_attn.py:27-29 and
 * :147-149). Rows with an empty band get o = 0 and lse = -inf.
 * Requires 0 <= band_lo < band_hi; band_hi >= T means unbounded.
 */
ttcd_status ttcd_band_attn_fwd(
    const void* q, const void* k, const void* v, void* o, float* lse, int B,
    int T, int Hq, int Hkv, int D, const int64_t q_stride[4],
    const int64_t k_stride[4], const int64_t v_stride[4],
    const int64_t o_stride[4], int band_lo, int band_hi, float sm_scale,
    ttcd_dtype dtype, void* stream);

/*
 * rescale_log2 (the calls below that take it; the two above use 8): the
 * online softmax keeps a reference row max and moves it, rescaling the
 * partial output, only when the probabilities against it could exceed
 * 2^rescale_log2: at head_dim 64 when a row's max exceeds it by more than
 * 2^rescale_log2, at head_dim 128 when a 64-key tile's probabilities over a
 * half row (32 keys) sum above 2^rescale_log2. Either way every probability
 * stays <= 2^rescale_log2. 8 (lazy) is the fastest. 0 keeps the exact running max of
 * the reference kernel (fused_dual_attn.py:100-107), whose numerics it then
 * follows: at config 1, 98.6 % (teacher) and 99.96 % (student) of the bf16
 * outputs are bit-identical to a CPU emulation of the reference kernel, vs
 * 58-61 % at 8, for ~8 % more time. Must lie in [0, 16] for BF16 and in
 * [0, 15] for F16 (probabilities reach 2^rescale_log2 and are rounded to the
 * input dtype before PV; f16 overflows at 65520), else
 * TTCD_ERR_INVALID_ARGUMENT.
 *
 * Cached prefill (Tq <= Tk): the same two calls for Tq new query rows against
 * Tk keys, the queries at absolute positions Tk - Tq .. Tk - 1 (the bottom-
 * right aligned causal mask of flash_attn_func with seqlen_q < seqlen_k, as
 * test/test_fused_dual_attn.py:275-293 specifies for fused_dual_window_attn,
 * where the reference kernel is a strict xfail). q, o_t, o_s, o: (B, Tq, Hq,
 * D); k, v: (B, Tk, Hkv, D); lse*: (B, Hq, Tq). Windows, bands and every
 * other argument as above; with Tq == Tk these are the calls above.
 */
ttcd_status ttcd_dual_window_attn_kv_fwd(
    const void* q, const void* k, const void* v, void* o_t, void* o_s,
    float* lse_t, float* lse_s, int B, int Tq, int Tk, int Hq, int Hkv, int D,
    const int64_t q_stride[4], const int64_t k_stride[4],
    const int64_t v_stride[4], const int64_t o_stride[4], int window_t,
    int window_s, float sm_scale, float rescale_log2, ttcd_dtype dtype,
    void* stream);

ttcd_status ttcd_band_attn_kv_fwd(
    const void* q, const void* k, const void* v, void* o, float* lse, int B,
    int Tq, int Tk, int Hq, int Hkv, int D, const int64_t q_stride[4],
    const int64_t k_stride[4], const int64_t v_stride[4],
    const int64_t o_stride[4], int band_lo, int band_hi, float sm_scale,
    float rescale_log2, ttcd_dtype dtype, void* stream);

/*
 * Packed variable-length sequences (flash-attention's varlen layout): the
 * same two calls on nseq sequences packed along the token axis. Sequence b
 * is rows cu_seqlens[b] .. cu_seqlens[b+1]-1 of q, k, v and the outputs;
 * every sequence is its own causal prefill (queries == keys). Replaces the
 * flash_attn_varlen_func(cu_seqlens_q=cu_seqlens, cu_seqlens_k=cu_seqlens,
 * ..., causal=True, window_size=(W-1, 0)) calls of the packed-batch path
 * (fla/layers/attn.py:255-270), which the reference's fused prefill declines
 * (_use_fast_prefill_path returns False for cu_seqlens,
 * custom_models/ipttcd/modeling_ipttcdv9.py:570-571).
 *   q, o_t, o_s, o: (total, Hq, D); k, v: (total, Hkv, D); strides are the
 *   token, head and d strides (d-stride 1). lse*: (Hq, total) fp32.
 *   cu_seqlens: device int32[nseq + 1], nondecreasing, cu_seqlens[0] = 0,
 *   cu_seqlens[nseq] = total. It is read on the device (no host sync); each
 *   sequence is clamped to rows [0, total) and to max_seqlen rows, so
 *   malformed offsets cannot cause an out-of-bounds access. Rows outside
 *   every sequence are not written.
 *   max_seqlen: the longest sequence (sizes the grid).
 * Windows, bands and every other argument as in the fixed-length calls
 * (window_t < 0: full causal within each sequence).
 */
ttcd_status ttcd_dual_window_attn_varlen_fwd(
    const void* q, const void* k, const void* v, void* o_t, void* o_s,
    float* lse_t, float* lse_s, const int32_t* cu_seqlens, int nseq,
    int max_seqlen, int total, int Hq, int Hkv, int D,
    const int64_t q_stride[3], const int64_t k_stride[3],
    const int64_t v_stride[3], const int64_t o_stride[3], int window_t,
    int window_s, float sm_scale, float rescale_log2, ttcd_dtype dtype,
    void* stream);

ttcd_status ttcd_band_attn_varlen_fwd(
    const void* q, const void* k, const void* v, void* o, float* lse,
    const int32_t* cu_seqlens, int nseq, int max_seqlen, int total, int Hq,
    int Hkv, int D, const int64_t q_stride[3], const int64_t k_stride[3],
    const int64_t v_stride[3], const int64_t o_stride[3], int band_lo,
    int band_hi, float sm_scale, float rescale_log2, ttcd_dtype dtype,
    void* stream);

/*
 * Exact log-sum-exp merge of two attention partials over disjoint key sets.
 * Replaces _lse_merge_kernel + the o_t[:, :WS] copy of
 * lse_dual_window_attn_fa3_fast (profiling/lse_dual_attn.py:106-131, :151-159).
 * Rows t < row_start: o_t = o_s (copied). Rows t >= row_start:
 *   lt = logaddexp(lse_s, lse_f); o_t = o_s*exp(lse_s-lt) + o_f*exp(lse_f-lt)
 * in fp32, rounded once to `dtype`. o_s, o_f, o_t: (B, T, H, D) sharing
 * o_stride; lse_s, lse_f: (B, H, T) contiguous fp32.
 */
ttcd_status ttcd_lse_merge_fwd(const void* o_s, const float* lse_s,
                               const void* o_f, const float* lse_f, void* o_t,
                               int B, int T, int H, int D, int row_start,
                               const int64_t o_stride[4], ttcd_dtype dtype,
                               void* stream);

/*
 * The LSE-combination variant in one call: o_s = the window_s call, o_t =
 * the exact log-sum-exp merge of o_s with the far band window_s <= i-j <
 * window_t. Replaces lse_dual_window_attn_fa3_fast (and
 * lse_dual_window_attn / _fa3, which compute the same thing;
 * profiling/lse_dual_attn.py:16-39, :74-99, :134-160), including its
 * o_t[:, :WS] = o_s[:, :WS] rows. Queries are the last Tq of Tk positions as
 * in the kv forms (Tq == Tk for a fresh prefill). Requires
 * 1 <= window_s < window_t (window_t < 0: full causal), as the reference
 * asserts (lse_dual_attn.py:20). Other arguments as in
 * ttcd_dual_window_attn_kv_fwd.
 * workspace: device scratch for the far-band partial and both LSEs,
 * 256-byte aligned. With workspace_bytes >=
 * ttcd_lse_dual_window_attn_workspace_bytes(...) the rows run in one pass;
 * a smaller workspace runs them in chunks that fit (same results, bit for
 * bit); TTCD_ERR_INVALID_ARGUMENT if it holds no row. The workspace is not
 * read before it is written and may be reused once the stream has passed
 * the call.
 */
size_t ttcd_lse_dual_window_attn_workspace_bytes(int B, int Tq, int Tk, int Hq, int D,
                                                 int window_s);
ttcd_status ttcd_lse_dual_window_attn_fwd(
    const void* q, const void* k, const void* v, void* o_t, void* o_s,
    int B, int Tq, int Tk, int Hq, int Hkv, int D,
    const int64_t q_stride[4], const int64_t k_stride[4],
    const int64_t v_stride[4], const int64_t o_stride[4],
    int window_t, int window_s, float sm_scale, float rescale_log2,
    ttcd_dtype dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Allocation-free form of ttcd_lse_dual_window_attn_fwd. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The workspace is a fixed device array inside the library,
 * ttcd_lse_dual_window_attn_noalloc_scratch_bytes() (64 MiB) per GPU, held
 * until the process ends; the call makes no allocation of its own. Rows run
 * in chunks that fit it, so any T works; TTCD_ERR_UNSUPPORTED when a single
 * query row does not fit (B * Hq * (2 * D + 8) bytes, i.e. B * Hq above
 * ~254,000 at D = 128). Results are bit-identical to
 * ttcd_lse_dual_window_attn_fwd. Every call on one GPU shares the array:
 * calls that overlap in time on one GPU (different streams with no ordering
 * between them) race; calls on one stream are safe. The first call on a
 * device resolves the array's address there (hipGetSymbolAddress), so make
 * that first call outside HIP graph capture; later calls can be captured
 * and replayed. Other arguments as in ttcd_lse_dual_window_attn_fwd.
 */
size_t ttcd_lse_dual_window_attn_noalloc_scratch_bytes(void);
ttcd_status ttcd_lse_dual_window_attn_noalloc_fwd(
    const void* q, const void* k, const void* v, void* o_t, void* o_s,
    int B, int Tq, int Tk, int Hq, int Hkv, int D,
    const int64_t q_stride[4], const int64_t k_stride[4],
    const int64_t v_stride[4], const int64_t o_stride[4],
    int window_t, int window_s, float sm_scale, float rescale_log2,
    ttcd_dtype dtype, void* stream);

/*
 * Chunk-local causal depthwise conv along C on the (N, C, D) layout.
 * Replaces causal_dwconv_chunked / _causal_dwconv_fwd
 * (profiling/fused_conv.py:24-61) and IPTTCDMLP._apply_ttt_conv with
 * ttt_conv_causal=True (custom_models/ipttcd/modeling_ipttcdv9.py:203-211).
 *   y[n,c,d] = sum_{j=0..K-1} w[d,j] * x[n, c-(K-1)+j, d]  (x = 0 for c < 0)
 * accumulated in fp32 as acc = fma(x, w, acc) for j = 0..K-1 from acc = +0,
 * then rounded once (RNE) to x_dtype. x, y: contiguous (N, C, D);
 * w: contiguous (D, K). 1 <= K <= 64.
 */
ttcd_status ttcd_causal_dwconv_chunked_fwd(const void* x, const void* w,
                                           void* y, int64_t N, int C, int D,
                                           int K, ttcd_dtype x_dtype,
                                           ttcd_dtype w_dtype, void* stream);

/*
 * Attention prologue: per-head RMSNorm of q and k (qk_norm) fused with the
 * rotary embedding, one read and one write of q and k. Replaces, at
 * profiling/patches.py:254-268, `q, k = attn.q_norm(q), attn.k_norm(k)`
 * (fla RMSNorm forward, fla/modules/layernorm.py:189-251) followed by
 * `q, k = attn.rotary(q, k, seqlen_offset=...)` (fla rotary_embedding_kernel,
 * non-interleaved, fla/modules/rotary.py:43-135).
 *
 * q: (B, T, Hq, D), k: (B, T, Hkv, D) of `dtype` (BF16 or F16), D in {64, 128};
 * q_out / k_out have the same shapes (they may alias q / k exactly).
 * *_stride[4] = element strides of (b, t, h, d); d-stride 1.
 * q_norm_w, k_norm_w: (D,) RMSNorm weights of w_dtype (BF16, F16 or F32), or
 * both NULL for rotary only. Per row: var = sum(x^2) / D,
 * y = (x / sqrt(var + eps)) * w rounded to dtype; then with x0 = y[:D/2],
 * x1 = y[D/2:], c/s = the table rows at position t + seqlen_offset:
 * out = [x0*c - x1*s, x0*s + x1*c] in fp32, rounded to dtype.
 * cos_table, sin_table: (table_rows, D/2) contiguous, `dtype`;
 * seqlen_offset + T <= table_rows.
 */
ttcd_status ttcd_qk_norm_rope_fwd(
    const void* q, const void* k, void* q_out, void* k_out,
    const void* q_norm_w, const void* k_norm_w, ttcd_dtype w_dtype, float eps,
    const void* cos_table, const void* sin_table, int table_rows, int B, int T,
    int Hq, int Hkv, int D, const int64_t q_stride[4],
    const int64_t k_stride[4], const int64_t q_out_stride[4],
    const int64_t k_out_stride[4], int seqlen_offset, ttcd_dtype dtype,
    void* stream);

/*
 * Rotary tables as fla's RotaryEmbedding builds them
 * (fla/modules/rotary.py:441-490, pos_idx_in_fp32): for t < rows and
 * i < half_dim, cos_table[t*half_dim + i] = cos(fp32(t) * inv_freq[i]) and
 * the same for sin, the product rounded once to fp32, the result rounded to
 * `dtype` (BF16 or F16). inv_freq: half_dim fp32 values in device memory
 * (the module's inv_freq buffer, rotary.py:418-425).
 */
ttcd_status ttcd_rope_table_fwd(void* cos_table, void* sin_table,
                                const float* inv_freq, int rows, int half_dim,
                                ttcd_dtype dtype, void* stream);

/*
 * Attention epilogue: the residual add + RMSNorm (prenorm) of the teacher and
 * the student attention outputs in one pass. Replaces, at
 * profiling/patches.py:296-298 (fuse_norm = True),
 *   student_output, _ = mlp_norm(student_attn_output, residual, True)
 *   hidden_states, residual = mlp_norm(teacher_attn_output, residual, True)
 * (fla RMSNorm forward with a residual, fla/modules/layernorm.py:189-251,
 * 715-764). All activations are (rows, hidden) contiguous of `dtype` (BF16 or
 * F16); norm_w: (hidden,) of w_dtype (BF16, F16 or F32). Per row, for
 * b in {t, s}: x_b = attn_b + residual in fp32, y_b = (x_b / sqrt(sum(x_b^2) /
 * hidden + eps)) * w rounded to dtype; hidden_out = y_t, student_out = y_s,
 * residual_out = x_t rounded to dtype. hidden % 8 == 0, hidden <= 2048.
 */
ttcd_status ttcd_dual_residual_rmsnorm_fwd(
    const void* attn_t, const void* attn_s, const void* residual,
    const void* norm_w, ttcd_dtype w_dtype, float eps, void* hidden_out,
    void* residual_out, void* student_out, int64_t rows, int hidden,
    ttcd_dtype dtype, void* stream);

/*
 * One RMSNorm over rows of `hidden` elements, in one of fla's two forward
 * forms (fla/modules/layernorm.py:189-251, 715-764):
 *   residual == NULL: y = RMSNorm(x) * w (plain; attn_norm at
 *     custom_models/ipttcd/modeling_ipttcdv9.py:627 and the final norm at
 *     :1112);
 *   residual != NULL: the prenorm form of :863, x' = f32(x) + f32(residual),
 *     residual_out = x' rounded, y = RMSNorm(x') * w with the variance of the
 *     unrounded x'.
 * Pass residual and residual_out both or neither. Numerics, layout and
 * limits as ttcd_dual_residual_rmsnorm_fwd.
 */
ttcd_status ttcd_rmsnorm_fwd(const void* x, const void* residual,
                             const void* norm_w, ttcd_dtype w_dtype, float eps,
                             void* y, void* residual_out, int64_t rows,
                             int hidden, ttcd_dtype dtype, void* stream);

/*
 * The block's closing residual add fused with the next block's plain RMSNorm
 * (custom_models/ipttcd/modeling_ipttcdv9.py:870 `hidden_states = residual +
 * hidden_states`, a bf16 torch add, then :627 `self.attn_norm(...)`):
 * sum_out = f32(x) + f32(residual) rounded to dtype, y = RMSNorm(sum_out) * w
 * computed from the ROUNDED sum, exactly as the two separate launches.
 * Numerics, layout and limits as ttcd_rmsnorm_fwd.
 */
ttcd_status ttcd_add_rmsnorm_fwd(const void* x, const void* residual,
                                 const void* norm_w, ttcd_dtype w_dtype,
                                 float eps, void* y, void* sum_out, int64_t rows,
                                 int hidden, ttcd_dtype dtype, void* stream);

/*
 * SwiGLU, fla's swiglu_fwd (fla/modules/activations.py:412-471, used by
 * swiglu and swiglu_linear in every MLP of the model): out = (g * s) * u
 * with s = 1 / (1 + exp(-g)), in fp32, rounded to dtype. Row-strided
 * (strides in elements, multiples of 8; cols % 8 == 0), so gate and up may
 * be the two halves of one (rows, 2*cols) GEMM output.
 */
ttcd_status ttcd_swiglu_fwd(const void* gate, const void* up, void* out,
                            int64_t rows, int cols, int64_t gate_stride,
                            int64_t up_stride, int64_t out_stride,
                            ttcd_dtype dtype, void* stream);

/*
 * The TTT MLP's feature pass in one launch. Replaces, in the TTT MLP's
 * forward (custom_models/ipttcd/modeling_ipttcdv9_lowcopy_scanfuse.py:48-70,
 * with the chunk-local conv of profiling/patches.py:411-432, and the diff of
 * the update loop at :117-120), the launches
 *   z = swiglu(gate_t, up_t); z_hat = swiglu(gate_s, up_s);
 *   z_target = conv_t(z); z_hat = conv_s(z_hat); diff = z_target - z_hat.
 * gu_t / gu_s: (B * nchunk * chunk, 2 * inter) teacher / student gate|up
 * rows (gate in columns [0, inter), up in [inter, 2 * inter)), row stride
 * gu_stride elements. conv_t / conv_s: (inter, kernel_size) depthwise causal
 * conv weights, chunk-local (zero history at each chunk start), or NULL for
 * no conv. Outputs (contiguous): z (rows, inter), z_hat (rows, inter) and
 * diff (B * (nchunk - 1) * chunk, inter) for every chunk but the last of each
 * batch row (NULL allowed when nchunk == 1). Every value is rounded to dtype
 * where the reference stores it; the convs accumulate in fp32 in tap order.
 * inter % 8 == 0, kernel_size <= 8.
 */
ttcd_status ttcd_ttt_features_fwd(const void* gu_t, const void* gu_s,
                                  int64_t gu_stride, const void* conv_t,
                                  const void* conv_s, ttcd_dtype w_dtype,
                                  int kernel_size, void* z, void* z_hat,
                                  void* diff, int B, int nchunk, int chunk,
                                  int inter, ttcd_dtype dtype, void* stream);

/*
 * The TTT MLP's update scan around its GEMMs (the group loop of
 * custom_models/ipttcd/modeling_ipttcdv9_lowcopy_scanfuse.py:121-172).
 *
 * ttcd_ttt_proj_beta_t_fwd: pdt[b*nupd + c, h, t] = pd[(b*nupd + c)*chunk + t, h]
 * * beta[b*beta_batch_stride + c*chunk + t], one rounding to dtype (the
 * dynamic learning rate, :126-127; beta NULL: no scaling), written transposed
 * per chunk, (B*nupd, H, chunk) contiguous, so that dW_c = pd_c^T z_hat_c
 * (:146-149) is one batched GEMM on contiguous operands. pd rows have stride
 * pd_stride elements.
 *
 * ttcd_ttt_scan_fwd: one update group. dw (nupd, H, inter) the group's chunk
 * updates, w_cur (H, inter) the weight at the group start. With acc_j the
 * running sum of dw[0..j] stored in dtype after every step (torch's GPU scan
 * of a bf16 tensor, :157) and cs_j = lr * acc_j rounded (:157), writes
 * steps_t[0] = w_cur^T and steps_t[s] = (w_cur + cs_{s-1})^T rounded for
 * s = 1 .. nsteps-1 (the chunk weights of :161-165), (nsteps, inter, H)
 * contiguous; and, if w_next is not NULL, w_next = w_cur + cs_{nupd-1}
 * rounded (:169-170). Requires nsteps <= nupd + 1. lr is the learning rate
 * as the dtype stores it. All additions and products in fp32, each rounded
 * once to dtype, as torch's bf16 ops round them.
 */
ttcd_status ttcd_ttt_proj_beta_t_fwd(const void* pd, int64_t pd_stride, const void* beta,
                                    int64_t beta_batch_stride, void* pdt, int B, int nupd,
                                    int chunk, int H, ttcd_dtype dtype, void* stream);
ttcd_status ttcd_ttt_scan_fwd(const void* dw, const void* w_cur, float lr, void* steps_t,
                              void* w_next, int nupd, int nsteps, int H, int inter,
                              ttcd_dtype dtype, void* stream);

/*
 * Host-only schedule check (no GPU work). Replays the attention kernels'
 * exact tile/phase schedule for one (b, h) slice of length T and adds, for
 * every (query i, key j) pair the kernel would fold into each output, one
 * to counts_near[i*T + j] (phase 1: student window, or the whole band of a
 * single-band call) and counts_far[i*T + j] (phase 2 of the dual kernel:
 * window_s <= i - j < window_t). Used by tests to prove every in-band pair
 * is visited exactly once. Set dual = 0 for the single-band schedule, in
 * which case window_s = band_lo and window_t = band_hi. gqa_group is the
 * query-head group size Hq/Hkv, which sets the workgroup geometry: 4
 * wavefronts of 16 rows (64 tokens) for an even group, of 32 rows (128
 * tokens) otherwise. The pairs are counted from the
 * per-slot words the kernel decodes (tile, action, band, mask, load bounds),
 * each first checked against the plan and the per-tile predicates.
 */
ttcd_status ttcd_attn_schedule_coverage(int T, int dual, int window_s,
                                        int window_t, int gqa_group,
                                        int32_t* counts_near,
                                        int32_t* counts_far);

#ifdef __cplusplus
}
#endif

#endif /* TTCD_H_ */
