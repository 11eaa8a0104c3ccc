/*
 * C ABI of the MI355X-native HSTU hot path (gfx950).
 *
 * Plain pointers and sizes only; every pointer is a device pointer unless it
 * says otherwise, and every entry point launches on the given HIP stream and
 * returns 0 (hipSuccess) or a hipError_t / HSTU_E* code without synchronising.
 * No entry point allocates device memory.
 *
 * Reference paths are relative to
 * recommendation_v4/hstu/generative_recommenders/ in zirui/mlperf-training.
 *
 * Layouts
 *   q, k, v, out, dq, dk, dv : jagged [T, H, D]; element (t, h, d) lives at
 *       base + t*row_stride + h*D + d (row_stride in elements, >= H*D), so
 *       column slices of a fused [T, 2048] UVQK buffer are accepted in place.
 *   seq_offsets               : int64 [B+1], exclusive cumsum of lengths.
 *   scales (FP8 inputs)       : fp32, scale(t, h) = s[t*scale_row_stride +
 *       h*scale_head_stride]; strides (0, 0) give one per-tensor scalar,
 *       (H, 1) per-token-per-head.  Dequantized value = e4m3 * scale.
 *   attn_bias                 : optional fp32 [H, 2R-1]; score(i, j) gets
 *       bias[h][clamp(i-j, -(R-1), R-1) + R-1] added before SiLU.  This bias
 *       is an extension: the reference has none (pass NULL for parity).
 */
#ifndef HSTU_MI355X_H_
#define HSTU_MI355X_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* input element types */
#define HSTU_DTYPE_BF16 0
#define HSTU_DTYPE_FP8_E4M3 1
#define HSTU_DTYPE_FP32 2 /* only where an entry point says so */
#define HSTU_DTYPE_FP8_E5M2 3 /* only where an entry point says so */

/* error codes beyond hipError_t (all negative) */
#define HSTU_E_BAD_ARG (-1)
#define HSTU_E_UNSUPPORTED (-2)
#define HSTU_E_SCRATCH_TOO_SMALL (-3) /* the call needs more than an allocation-free entry point's scratch */

/* Library version / self-description; host pointer to a static string. */
const char* hstu_version(void);

/*
 * Jagged causal SiLU attention, forward:
 *   out_i = sum_{valid j} silu(alpha * q_i.k_j [+ bias]) / N * v_j
 * (N = max_seq_len).  Output is bf16 for both input types.
 * Mask options follow _get_valid_attn_mask: num_targets (int32 [B], nullable),
 * max_attn_len, contextual_seq_len (0 = off).
 * Replaces: triton_hstu_attention_fwd, ops/triton/triton_hstu_attention.py:3166-3295
 *           (launch of _hstu_attn_fwd, grid at :3247-3250), and the FlyDSL
 *           forward launches fn(q, k, v, out, cu, batch, m_blocks, 1/N[, qkv_scale])
 *           at ops/flydsl/hstu_flydsl_mha.py:2045-2046 and :2428-2429.
 */
int hstu_attn_fwd(int dtype,
                  const void* q, const void* k, const void* v,
                  int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                  const float* q_scale, const float* k_scale, const float* v_scale,
                  int64_t scale_row_stride, int64_t scale_head_stride,
                  const int64_t* seq_offsets, int B, int H, int D, int max_seq_len,
                  float alpha,
                  const int32_t* num_targets, int max_attn_len, int contextual_seq_len,
                  const float* attn_bias, int bias_R,
                  void* out, int64_t out_row_stride,
                  void* workspace, int64_t workspace_bytes, int64_t total_tokens,
                  hipStream_t stream);

/*
 * Device workspace hstu_attn_fwd needs (bytes, > 0): the per-call block
 * schedule (which XCD runs which (sequence, head) block).  total_tokens = T
 * = seq_offsets[B].  Returns -1 for bad sizes.  The reference's launchers
 * take no workspace (ops/flydsl/hstu_flydsl_mha.py:2036-2046).
 */
int64_t hstu_attn_fwd_workspace_bytes(int dtype, int64_t total_tokens, int B, int H, int D, int max_seq_len);

/*
 * FP8 P.V forward: hstu_attn_fwd on e4m3 q, k, v (D = 128, causal mask only:
 * num_targets must be null, max_attn_len and contextual_seq_len 0, else
 * HSTU_E_UNSUPPORTED) with the SiLU output rounded to e4m3 before P.V:
 * P8 = e4m3(sat(P' * pv_scale * r_k)), P' = -log2(e) silu(score), and P.V
 * on the e4m3 MFMA with V raw; out = sum_k P8 v8_k 2^E(k) * (-ln 2) /
 * (pv_scale * max_seq_len) [* v_scale].  With one per-tensor scale (scale
 * strides 0) r_k = 1 and v_scale rides on the output; with [T, H] scales
 * r_k = v_scale(k) 2^-E(k), E(k) the frexp exponent of the largest V scale
 * among the keys of k's group (64-key tiles from the sequence start, split by
 * bit 4 of the key's index in the tile).  pv_scale in (0, 448); the
 * reference's default is 10.04.  Workspace as hstu_attn_fwd (e4m3 dtype).
 * max_seq_len above hstu_attn_fwd_fp8_pv_max_seq_len() (a per-key table in
 * LDS outgrows the CU's 160 KiB) returns HSTU_E_UNSUPPORTED before any launch.
 * Replaces: the FlyDSL e4m3 forward with pv="k128" (DLRM_HSTU_FP8_FWD_PV=1),
 * ops/flydsl/hstu_flydsl_mha.py:2199-2330, ops/flydsl/hstu_fwd.py:253-283.
 */
int hstu_attn_fwd_fp8_pv(const void* q, const void* k, const void* v,
                         int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                         const float* q_scale, const float* k_scale, const float* v_scale,
                         int64_t scale_row_stride, int64_t scale_head_stride,
                         const int64_t* seq_offsets, int B, int H, int D, int max_seq_len,
                         float alpha,
                         const int32_t* num_targets, int max_attn_len, int contextual_seq_len,
                         const float* attn_bias, int bias_R, float pv_scale,
                         void* out, int64_t out_row_stride,
                         void* workspace, int64_t workspace_bytes, int64_t total_tokens,
                         hipStream_t stream);
/*
 * The largest max_seq_len hstu_attn_fwd_fp8_pv serves (a multiple of 64).
 * Replaces: the reference's shape gate that declines a call with a reason
 * before any launch, ops/flydsl/hstu_flydsl_mha.py:311-354.
 */
int hstu_attn_fwd_fp8_pv_max_seq_len(void);

/*
 * hstu_attn_fwd without a workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  The same kernels and
 * results as hstu_attn_fwd; the block schedule goes to a static device array
 * of HSTU_ATTN_FWD_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends.  A call needs hstu_attn_fwd_workspace_bytes(...) of it, about
 * 8 * B * (H + 1) bytes (B <= 6 500 sequences at H = 4); a larger call
 * returns HSTU_E_SCRATCH_TOO_SMALL before any launch.  Calls no hipMalloc / hipFree.  All calls on one GPU share its
 * array: calls that overlap on one GPU (concurrent streams) race, so
 * serialise them.
 */
#define HSTU_ATTN_FWD_NOALLOC_SCRATCH_BYTES (256 * 1024)
int hstu_attn_fwd_noalloc(int dtype,
                          const void* q, const void* k, const void* v,
                          int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                          const float* q_scale, const float* k_scale, const float* v_scale,
                          int64_t scale_row_stride, int64_t scale_head_stride,
                          const int64_t* seq_offsets, int B, int H, int D, int max_seq_len,
                          float alpha,
                          const int32_t* num_targets, int max_attn_len, int contextual_seq_len,
                          const float* attn_bias, int bias_R,
                          void* out, int64_t out_row_stride,
                          int64_t total_tokens, hipStream_t stream);

/*
 * Backward of hstu_attn_fwd.  Writes dq, dk, dv (bf16, caller-owned, may be
 * strided views) completely -- no accumulation into existing contents, so no
 * zero-fill is needed -- and, if dbias != NULL, overwrites dbias (fp32
 * [H, 2R-1]) with the bias gradient.  Gradients are with respect to the
 * dequantized q, k, v.  Deterministic, bias gradient included: no atomics;
 * each 128-query dQ block writes its own row of bias-gradient sums and the
 * rows are summed in a fixed order.  With a bias, the dQ kernels keep one
 * histogram per wave in LDS: 16 R bytes (causal mask) or 16 (2R - 1) bytes
 * (other masks) beyond their tiles; a bias_R past the CU's 160 KiB returns
 * HSTU_E_UNSUPPORTED before any launch.
 * Replaces: triton_hstu_attention_bwd, ops/triton/triton_hstu_attention.py:3298-3410
 *           (mutates_args dq/dk/dv), and the FlyDSL backward launch
 *           fn(q, k, v, dout, dk, dv, dq_slot, cu, batch, n_blocks, 1/N, qkv_scale)
 *           at ops/flydsl/hstu_flydsl_mha.py:1707-1723.
 */
int hstu_attn_bwd(int dtype,
                  const void* dout, int64_t dout_row_stride,
                  const void* q, const void* k, const void* v,
                  int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                  const float* q_scale, const float* k_scale, const float* v_scale,
                  int64_t scale_row_stride, int64_t scale_head_stride,
                  const int64_t* seq_offsets, int B, int H, int D, int max_seq_len,
                  float alpha,
                  const int32_t* num_targets, int max_attn_len, int contextual_seq_len,
                  const float* attn_bias, int bias_R,
                  void* dq, void* dk, void* dv,
                  int64_t dq_row_stride, int64_t dk_row_stride, int64_t dv_row_stride,
                  float* dbias,
                  void* workspace, int64_t workspace_bytes, int64_t total_tokens,
                  hipStream_t stream);

/*
 * Device workspace the backward needs (bytes): the block schedule; with a
 * bias (bias_R > 0; 0 = no bias) a pre-clamped copy of the bias rows, one
 * bias-gradient row of 2R - 1 floats per dQ block (ceil(T/128) + B per head)
 * and 64 chunk sums of them; the per-sequence dQ block prefix; for e4m3
 * inputs an exact bf16 copy of q; the dS tiles (8 KiB per 128-key x 32-query tile, bounded by
 * 2 (ceil(N/128) + 1) (ceil(T/128) + B) H tiles).  total_tokens = T = seq_offsets[B].  Returns -1 for bad sizes.  The
 * caller allocates it (the reference's FlyDSL backward likewise takes its
 * dq-split workspace from the caller, ops/flydsl/hstu_flydsl_mha.py:1674-1741).
 * hstu_attn_bwd_dkdv and hstu_attn_bwd_dq must be given the same workspace,
 * dkdv first: with the causal mask (no num_targets, window or contextual
 * prefix) dkdv leaves the bf16 dS tiles there and dq contracts them with K.
 */
int64_t hstu_attn_bwd_workspace_bytes(int dtype, int64_t total_tokens, int B, int H, int D, int max_seq_len,
                                      int bias_R);

/*
 * Full-FP8 backward (causal mask only; D = 128): e4m3 q, k, v as for
 * hstu_attn_bwd, and the upstream gradient as the block quantizer leaves it
 * -- dout8 e4m3 [T, H, D] (row stride dout_row_stride bytes, 16-byte aligned
 * rows) and dout_e8 uint8 [T, H] = 127 - e with dO = dout8 * 2^-e per
 * (sequence, head, 32-token group) (hstu_quantize_do_e4m3_blk).  All five
 * products run on the e4m3 MFMA: P and dS are cast to e4m3 with
 * power-of-two pre-scales, e4m3(silu / N * 2^p8_scale_log2) and
 * e4m3(dS * 2^ds8_scale_log2), and the dO group scales are applied by the
 * MFMA's E8M0 block-scale operands.  The reference's pre-scales are
 * N-relative: p8_scale_log2 = ceil(log2 N) + K_SSC (K_SSC = 3,
 * DLRM_HSTU_FP8_BWD_FULL_SSC_K) and ds8_scale_log2 = ceil(log2 N) + K_DSC
 * (K_DSC = -3 by default, DLRM_HSTU_FP8_BWD_FULL_DSC_K; -5 in the
 * production gin), or an absolute *_LOG2; both within [-64, 64] and
 * p8_scale_log2 <= ceil(log2 N) + 9 (the SiLU's upper-only clamp), else
 * HSTU_E_BAD_ARG.  dS passes from the dK/dV kernel to the
 * dQ kernel as e4m3 tiles in the workspace.  Writes dq, dk, dv (bf16) and,
 * if dbias != NULL, the bias gradient (computed from the e4m3 dS); every
 * output is bitwise deterministic (the bias gradient as hstu_attn_bwd's).
 * Replaces: flydsl_hstu_attention_bwd under DLRM_HSTU_FP8_BWD_FULL
 *           (ops/flydsl/hstu_flydsl_mha.py:1330-1394 dO contract, :1351-1370
 *           pre-scales, :1674-1741 dq split; ops/flydsl/hstu_bwd_dkdv.py:356-403;
 *           dlrm_v4/train/gin/yambda_5b.gin:3764-3799 for K_DSC = -5).
 */
int64_t hstu_attn_bwd_fp8_workspace_bytes(int64_t total_tokens, int B, int H, int D, int max_seq_len,
                                          int bias_R);
int hstu_attn_bwd_fp8(const void* dout8, const void* dout_e8, int64_t dout_row_stride,
                      const void* q, const void* k, const void* v,
                      int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                      const float* q_scale, const float* k_scale, const float* v_scale,
                      int64_t scale_row_stride, int64_t scale_head_stride,
                      const int64_t* seq_offsets, int B, int H, int D, int max_seq_len,
                      float alpha, int p8_scale_log2, int ds8_scale_log2,
                      const float* attn_bias, int bias_R,
                      void* dq, void* dk, void* dv,
                      int64_t dq_row_stride, int64_t dk_row_stride, int64_t dv_row_stride,
                      float* dbias, void* workspace, int64_t workspace_bytes, int64_t total_tokens,
                      hipStream_t stream);
/*
 * Its two halves, same arguments, run in order on one stream with one
 * workspace: _dkdv writes dk, dv and leaves the e4m3 dS tiles (and the block
 * schedule, tile prefixes, pre-clamped bias rows and scale maxima) in the
 * workspace; _dq reads them and writes dq and dbias.
 */
int hstu_attn_bwd_fp8_dkdv(const void* dout8, const void* dout_e8, int64_t dout_row_stride,
                           const void* q, const void* k, const void* v,
                           int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                           const float* q_scale, const float* k_scale, const float* v_scale,
                           int64_t scale_row_stride, int64_t scale_head_stride,
                           const int64_t* seq_offsets, int B, int H, int D, int max_seq_len,
                           float alpha, int p8_scale_log2, int ds8_scale_log2,
                           const float* attn_bias, int bias_R,
                           void* dq, void* dk, void* dv,
                           int64_t dq_row_stride, int64_t dk_row_stride, int64_t dv_row_stride,
                           float* dbias, void* workspace, int64_t workspace_bytes, int64_t total_tokens,
                           hipStream_t stream);
int hstu_attn_bwd_fp8_dq(const void* dout8, const void* dout_e8, int64_t dout_row_stride,
                         const void* q, const void* k, const void* v,
                         int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                         const float* q_scale, const float* k_scale, const float* v_scale,
                         int64_t scale_row_stride, int64_t scale_head_stride,
                         const int64_t* seq_offsets, int B, int H, int D, int max_seq_len,
                         float alpha, int p8_scale_log2, int ds8_scale_log2,
                         const float* attn_bias, int bias_R,
                         void* dq, void* dk, void* dv,
                         int64_t dq_row_stride, int64_t dk_row_stride, int64_t dv_row_stride,
                         float* dbias, void* workspace, int64_t workspace_bytes, int64_t total_tokens,
                         hipStream_t stream);

/*
 * The two halves of hstu_attn_bwd, same arguments: hstu_attn_bwd_dkdv writes
 * dk and dv only (dq may be NULL); hstu_attn_bwd_dq writes dq and dbias only
 * (dk, dv may be NULL).  Each writes its own parts of the shared workspace,
 * so run them in order on one stream, dkdv first.  The reference launches its
 * backward in the same two parts when the dq-split is armed: the fused dK/dV
 * kernel, then dq from the stored ds tiles (ops/flydsl/hstu_flydsl_mha.py:1707-1740,
 * ops/flydsl/hstu_dq_split.py:348).  Here too, with the causal mask dq
 * contracts the dS tiles that dkdv left in the workspace with K (it cannot
 * run without them); only the generic masks (num_targets, window, contextual
 * prefix) make dq recompute the score tiles itself.
 */
int hstu_attn_bwd_dkdv(int dtype, const void* dout, int64_t dout_row_stride, const void* q, const void* k,
                       const void* v, int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                       const float* q_scale, const float* k_scale, const float* v_scale,
                       int64_t scale_row_stride, int64_t scale_head_stride, const int64_t* seq_offsets,
                       int B, int H, int D, int max_seq_len, float alpha, const int32_t* num_targets,
                       int max_attn_len, int contextual_seq_len, const float* attn_bias, int bias_R,
                       void* dq, void* dk, void* dv, int64_t dq_row_stride, int64_t dk_row_stride,
                       int64_t dv_row_stride, float* dbias, void* workspace, int64_t workspace_bytes,
                       int64_t total_tokens, hipStream_t stream);
int hstu_attn_bwd_dq(int dtype, const void* dout, int64_t dout_row_stride, const void* q, const void* k,
                     const void* v, int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                     const float* q_scale, const float* k_scale, const float* v_scale,
                     int64_t scale_row_stride, int64_t scale_head_stride, const int64_t* seq_offsets,
                     int B, int H, int D, int max_seq_len, float alpha, const int32_t* num_targets,
                     int max_attn_len, int contextual_seq_len, const float* attn_bias, int bias_R,
                     void* dq, void* dk, void* dv, int64_t dq_row_stride, int64_t dk_row_stride,
                     int64_t dv_row_stride, float* dbias, void* workspace, int64_t workspace_bytes,
                     int64_t total_tokens, hipStream_t stream);

/*
 * FP8 e4m3 projection GEMM: C[m][n] = epilogue(sum_k A[m][k] * W[n][k]).
 *   A: [M, K] e4m3 row-major, lda bytes; a_scale: a_scale_mode 0 -> one
 *      fp32 scalar, 1 -> [M] per row.
 *   W: [N, K] e4m3 row-major (the transposed weight), ldw bytes; w_scale:
 *      w_scale_mode 0 -> scalar, 1 -> [N] per output column.
 *   epilogue: v = acc * sa * sw [+ bias[n] (bf16 [N])]; v = silu(v) for
 *      silu_begin <= n < silu_end; [+ residual[m][n] (bf16, ldr elements)];
 *      out_dtype HSTU_DTYPE_BF16 -> bf16 C, HSTU_DTYPE_FP8_E4M3 -> e4m3 of
 *      clamp(v / out_scale[0], +-448).  ldc in elements.
 *   N % 128 == 0, K % 128 == 0; any M (rows past M are not touched).
 * Replaces: k512_fp8_gemm_e4m3_bias_N{N}(A, B, C, bias, sa, sb, M, stream),
 *           ops/hip/k512_fp8_gemm.cu:555-578 (e4m3 out, K=512); the K=1536
 *           residual add-mm k1536_fp8_addmm_res_bf16_N512, ops/hip/k1536_fp8_addmm.cu:435-441;
 *           and the hipBLASLt scaled GEMMs behind scaled_addmm_fp8_preq /
 *           scaled_mm_fp8_out_preq (ops/triton/triton_fp8.py:1756, 2409).
 */
int hstu_fp8_gemm_rowcol(const void* A, int64_t lda, const void* W, int64_t ldw,
                         const float* a_scale, int a_scale_mode,
                         const float* w_scale, int w_scale_mode,
                         const void* bias, const void* residual, int64_t ldr,
                         void* C, int64_t ldc, int out_dtype, const float* out_scale,
                         int M, int N, int K, int silu_begin, int silu_end,
                         hipStream_t stream);

/*
 * The same GEMM with the A format explicit: a_dtype HSTU_DTYPE_FP8_E4M3 is
 * hstu_fp8_gemm_rowcol; HSTU_DTYPE_FP8_E5M2 takes A in e5m2 (a backward
 * gradient) against the e4m3 W, bf16 output, no residual -- the FP8 dgrad
 * dX = dY8 . W8^T with per-tensor scales.
 * Replaces: output_projection_dgrad's torch._scaled_mm(gradient_e5m2, weight_e4m3.t(),
 *           scale_a, scale_b, out_dtype=bf16), ops/triton/bwd_fp8.py:1347-1395.
 */
int hstu_fp8_gemm(int a_dtype, const void* A, int64_t lda, const void* W, int64_t ldw, const float* a_scale,
                  int a_scale_mode, const float* w_scale, int w_scale_mode, const void* bias, const void* residual,
                  int64_t ldr, void* C, int64_t ldc, int out_dtype, const float* out_scale, int M, int N, int K,
                  int silu_begin, int silu_end, hipStream_t stream);

/*
 * bf16 projection GEMM on the same tile kernel: C[m][n] = epilogue(sum_k
 * A[m][k] W[n][k]), A [M, K] and W [N, K] row-major bf16 (lda, ldw, ldc, ldr
 * in elements), fp32 accumulate, epilogue as hstu_fp8_gemm without scales
 * (+ bias[n], SiLU on [silu_begin, silu_end), + residual), bf16 C.
 * N % 128 == 0, K % 64 == 0, 16-byte aligned A / W rows.  Each output row
 * depends on its own A row only (no M-dependent split), so a row's result
 * does not change with the batch it is computed in.
 * Replaces: the layer's bf16 GEMMs on the host BLAS -- the projection dgrads
 *           torch.mm(dout, output_weight.t()) (ops/triton/triton_hstu_linear.py:5588)
 *           and the UVQK dgrad, and the bf16 UVQK projection
 *           maybe_triton_addmm_fwd -> torch.addmm on ROCm (ops/triton/triton_addmm.py:1756-1767).
 */
int hstu_bf16_gemm(const void* A, int64_t lda, const void* W, int64_t ldw, const void* bias, const void* residual,
                   int64_t ldr, void* C, int64_t ldc, int M, int N, int K, int silu_begin, int silu_end,
                   hipStream_t stream);

/*
 * One-pass FP8 cast with the input's amax: out[i] = fp8(clamp(x[i] *
 * inv_scale[0], +-limit)) (out_dtype e4m3 or e5m2, round to nearest even)
 * over n contiguous bf16 / fp32 elements (n % 32 == 0, 16-byte aligned), and
 * partial_amax[b] = max |x| over elements [8192 b, 8192 (b + 1)), before
 * scaling; hstu_cast_fp8_amax_partials(n) partials.  inv_scale stays on
 * the device (no host sync).
 * Replaces: quantize_row_major / _quantize_amax_kernel, ops/triton/bwd_fp8.py:194-217, 827-866.
 */
int64_t hstu_cast_fp8_amax_partials(int64_t n);
int hstu_cast_fp8_amax(int in_dtype, const void* x, int64_t n, const float* inv_scale, int out_dtype, float limit,
                       void* out, float* partial_amax, int64_t partial_count, hipStream_t stream);

/*
 * e4m3 at unit margin with the scale derived on the device (two launches):
 * scale_out[0] = max(amax |x|, 1e-30) * fp32(1 / 448), out = e4m3(clamp(x *
 * (1 / scale), +-448)), 1 / scale correctly rounded; x bf16 / fp32 (in_dtype),
 * n > 0, n % 32 == 0, 16-byte aligned; partial: hstu_cast_fp8_amax_partials(n)
 * fp32 of scratch.  Bitwise equal to the torch expression it replaces.
 * Replaces: quantize_weight, ops/triton/bwd_fp8.py:1157-1175 (the
 *           DLRM_HSTU_FP8_BWD_HELPERS_FUSED form :1178-1190 is likewise one
 *           amax launch + one cast launch).
 */
int hstu_quantize_e4m3_unit(int in_dtype, const void* x, int64_t n, void* out, float* scale_out, float* partial,
                            int64_t partial_count, hipStream_t stream);

/*
 * One call's update of a delayed-scale gradient site in one launch; state
 * (device fp32 [4]) = [scale, 1 / scale, window peak, overflowed calls].
 * a = max of amax_values[0 .. count) (a cast's partials, or one amax; NaN
 * propagates); when live, state[3] += (a > state[0] * limit); state[2] =
 * max(state[2], a); snapshot (nullable) <- state[0]; when roll, state[0] =
 * max(state[2], 1e-30) * factor, state[1] = 1 / state[0], state[2] = 0.
 * Replaces: the partial-amax reduce, note_clipping, accumulate, the decode
 *           scale snapshot and the publish of the reference's _SiteScale,
 *           ops/triton/bwd_fp8.py:869-1154 (fused as in :1178-1190).
 */
int hstu_fp8_site_update(const float* amax_values, int count, float* state, float limit, int live, int roll,
                         float factor, float* snapshot, hipStream_t stream);

/*
 * One read of a row-major bf16 gradient x [rows, cols] (row stride ldx,
 * cols % 256 == 0) -> out [rows_out, cols] contiguous fp8 (out_dtype e4m3 or
 * e5m2) = fp8(clamp(x * inv_scale[0], +-limit)), RNE, with rows in
 * [rows, rows_out) written as zero (K padding for a token-contracting GEMM);
 * amax[0] = max |x| and colsum[c] = fp32 sum over rows of x[:, c] (the bias
 * gradient, of the unquantized input; a fixed reduction order: 512-row
 * stripes, then the stripes).  workspace: at least
 * hstu_cast_fp8_amax_colsum_workspace_bytes(rows, cols) bytes of device
 * memory (the per-stripe partials).  inv_scale stays on the device.
 * Replaces: quantize_amax_colsum / _quantize_amax_colsum_kernel,
 *           ops/triton/bwd_fp8.py:378-434, 608-692.
 */
int64_t hstu_cast_fp8_amax_colsum_workspace_bytes(int64_t rows, int64_t cols);
int hstu_cast_fp8_amax_colsum(const void* x, int64_t ldx, int64_t rows, int64_t cols, const float* inv_scale,
                              int out_dtype, float limit, void* out, int64_t rows_out, float* colsum, float* amax,
                              void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Weight gradient over the token axis from row-major (one token per row)
 * operands: out[n1][n2] = sa * sb * sum_{t < T} A[t][n1] * B[t][n2], fp32
 * accumulation, out bf16 (HSTU_DTYPE_BF16) or fp32 (HSTU_DTYPE_FP32) with row
 * stride ldo.  A [T, N1] (row stride lda elements), B [T, N2] (ldb): both
 * HSTU_DTYPE_BF16, or A HSTU_DTYPE_FP8_E4M3 with B HSTU_DTYPE_FP8_E4M3 or
 * HSTU_DTYPE_FP8_E5M2 (the FP8 backward's activation x gradient); N1, N2
 * multiples of 256; rows 16-byte aligned.  scale_a /
 * scale_b: one fp32 on the device each, or NULL for 1.  The tokens are split
 * over `split` ranges (<= 0: about one workgroup per CU); the per-split fp32
 * partials go to workspace (hstu_wgrad_workspace_bytes bytes, 0 for one
 * split) and are summed in a fixed order (bitwise reproducible).  T = 0
 * writes zeros.  hstu_wgrad_split gives the split actually used.
 * colsum_b (bf16 operands only; NULL to skip): fp32 [N2], 16-byte aligned,
 * receives sum_t B[t][n2] (unscaled) -- the bias gradient of a projection
 * whose output gradient is B -- from the same pass.
 * Replaces: dw = torch.mm(x.t(), dz) of triton_addmm_bwd,
 *           ops/triton/triton_addmm.py:1737-1750, and the output projection's
 *           torch.mm(y.t(), dout), ops/triton/triton_hstu_linear.py; fp8_wgrad
 *           (fp8 operands, the same split-K scheme), ops/triton/fp8_wgrad.py:27-160.
 */
int hstu_wgrad_split(int64_t T, int N1, int N2, int split);
int64_t hstu_wgrad_workspace_bytes(int64_t T, int N1, int N2, int split);
int hstu_wgrad(int a_dtype, const void* A, int64_t lda, int b_dtype, const void* B, int64_t ldb, int64_t T, int N1,
               int N2, const float* scale_a, const float* scale_b, void* out, int64_t ldo, int out_dtype,
               float* colsum_b, int split, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * e4m3 quantization of bf16 rows in groups of `group` consecutive elements:
 * scale = amax/448 per group (1/448 for an all-zero group), written to
 * scale_out[row * (cols/group) + group_index]; out = e4m3(clamp(x/scale,
 * +-448)).  With scale_in != NULL, that single per-tensor scale is used and
 * nothing is written to scale_out.  group % 8 == 0, group <= 4096.
 * [T, H, D] per-(token, head): rows=T, cols=H*D, group=D.  Per-row: group=cols.
 * Replaces: quantize_with_scale / calibrated_scale,
 *           ops/triton/triton_fp8.py:396-413, 760-781.
 */
int hstu_quantize_e4m3_rows(const void* x, int64_t ldx, int rows, int cols, int group,
                            const float* scale_in, void* out, int64_t ldo, float* scale_out,
                            hipStream_t stream);

/*
 * LayerNorm * U * dropout of the output block, and the weighted LayerNorm.
 * Rows of x, u: bf16 [rows, D] with row strides (elements); D = 256 or 512.
 * weight, bias: [D], fp32 (param_dtype HSTU_DTYPE_FP32) or bf16
 * (HSTU_DTYPE_BF16, the parameters' own dtype, converted exactly on load),
 * 16-byte aligned.
 * mean, rstd: fp32 [rows] (written by the forward).
 * mul_u_act: 0 none (ln * u), 1 silu (ln * silu(u)), 2 sigmoid.
 * u == NULL: plain weighted LayerNorm, y = ln (concat_u, mul_u_act, silu_u
 * ignored).
 * Output columns, in order: [u' if concat_u][x if concat_x][ln * m(u)], each
 * D wide; u' = silu(u) when silu_u.  Dropout (training && ratio > 0) zeroes or
 * scales each element by fp32(1 / fp32(1 - ratio)) with an int8 keep mask
 * [rows, D] (row stride ldm): bit 0 = y, then x (if concat_x), then u (if
 * concat_u).  The mask is Philox4x32-10 (key = seed's two 32-bit words) at
 * counter p * nmasks * BLOCK_D + j * BLOCK_D + col for mask j of row group p
 * (BLOCK_D = next power of two of D); mask16 = 0: groups of 4 rows, word i
 * decides row i, kept iff (x ^ (x >> 31)) > keep_above(ratio); mask16 = 1:
 * groups of 8 rows, word i's low / high half decides row i / i + 4, kept iff
 * half >= round(ratio * 65536).
 * Replaces: _create_dropout_mask, ops/triton/triton_hstu_linear.py:2547-2600
 *           (_generate_random_mask :331-375, _generate_random_mask16 :428-470).
 */
int hstu_dropout_mask(int rows, int D, int num_masks, int mask16, float dropout_ratio, uint64_t seed,
                      void* mask, int64_t ldm, hipStream_t stream);

/*
 * Forward.  y: bf16 or e4m3 (out_dtype) [rows, ncols * D] with row stride
 * ldy; e4m3 stores e4m3(clamp(value * inv_scale, +-448)).  out_scale (device
 * fp32, nullable): when given, the e4m3 output uses 1 / out_scale[0], read on
 * the device, instead of inv_scale -- the layer's per-tensor dequantization
 * scale never travels to the host.  With dropout the keep mask is generated
 * (as by hstu_dropout_mask) and written to `mask`.
 * Replaces: triton_layer_norm_mul_dropout_fwd, triton_hstu_linear.py:3034-3146
 *           (kernels _ln_mul_dropout_fwd :1429-1563, _ln_mul_dropout_fwd_rng
 *           :529-700); triton_weighted_layer_norm_fwd,
 *           ops/triton/triton_layer_norm.py:1668-1740 (u == NULL).
 */
int hstu_ln_mul_fwd(const void* x, int64_t ldx, const void* u, int64_t ldu,
                    const void* weight, const void* bias, int param_dtype, float eps, int rows, int D,
                    int mul_u_act, int silu_u, int concat_u, int concat_x,
                    int training, float dropout_ratio, uint64_t seed, int mask16,
                    void* mask, int64_t ldm,
                    void* y, int64_t ldy, int out_dtype, float inv_scale, const float* out_scale,
                    float* mean, float* rstd, hipStream_t stream);

/* Workspace of hstu_ln_mul_bwd (per-block dweight / dbias partials). */
int64_t hstu_ln_mul_bwd_workspace_bytes(int rows, int D);

/*
 * Backward.  dy: bf16 [rows, ncols * D] (the gradient of y, in y's column
 * order); mask as written by the forward (NULL: no dropout).  Writes dx, du
 * (bf16, du only with u), dweight and dbias (fp32 [D], deterministic: fixed
 * summation order) and, when y != NULL, the bf16 forward output recomputed
 * (for the output projection's weight gradient).  dres (NULL: none): a bf16
 * [rows, D] gradient from a residual branch of x, added to dx before its
 * rounding (not with concat_x or a mask).
 * Replaces: triton_layer_norm_mul_dropout_bwd, triton_hstu_linear.py:3689-3747
 *           (kernel _ln_mul_dropout_bwd_dx_du_rng :1566-1760, finalize
 *           _lnmd_bwd_finalize :3402-3431); triton_weighted_layer_norm_bwd,
 *           ops/triton/triton_layer_norm.py:3574-3640 (u == NULL, no residual).
 */
int hstu_ln_mul_bwd(const void* dy, int64_t lddy, const void* x, int64_t ldx,
                    const void* u, int64_t ldu, const void* weight, const void* bias, int param_dtype,
                    const float* mean, const float* rstd, int rows, int D,
                    int mul_u_act, int silu_u, int concat_u, int concat_x,
                    float dropout_ratio, const void* mask, int64_t ldm,
                    void* dx, int64_t lddx, void* du, int64_t lddu, void* y, int64_t ldy,
                    const void* dres, int64_t lddres,
                    float* dweight, float* dbias, void* workspace, int64_t workspace_bytes,
                    hipStream_t stream);

/* Workspace of hstu_outproj_ln_bwd (per-workgroup dweight / dbias partials). */
int64_t hstu_outproj_ln_bwd_workspace_bytes(int rows);

/*
 * The output projection's FP8 dgrad fused with the LN * U * dropout backward
 * of the [u' | x | y] concat (D = 512, W [1536, 512]): dy = bf16(g8 . w8^T *
 * g_scale * w_scale) is formed 64 rows at a time on chip and consumed by the
 * row backward, never stored.  g8: e5m2 [rows, 512] (ldg bytes); w8: e4m3
 * [1536, 512] (ldw bytes); g_scale, w_scale: fp32 device scalars.  The other
 * arguments and outputs are hstu_ln_mul_bwd's (concat_u = concat_x = 1, no
 * recomputed y): dx and du equal the unfused hstu_fp8_gemm (e5m2 dgrad) +
 * hstu_ln_mul_bwd bit for bit; dweight / dbias are deterministic (fixed
 * summation order, a different one than the unfused path's).
 * Replaces: l11_outproj_lnmd_bwd_launch,
 *           ops/hip/l11_outproj_lnmd.cu:906-910 (host finalize of its
 *           partials: triton_hstu_linear.py:5410-5470).
 */
int hstu_outproj_ln_bwd(const void* g8, int64_t ldg, const float* g_scale, const void* w8, int64_t ldw,
                        const float* w_scale, const void* x, int64_t ldx, const void* u, int64_t ldu,
                        const void* weight, const void* bias, int param_dtype, const float* mean,
                        const float* rstd, int rows, int D, int mul_u_act, int silu_u, float dropout_ratio,
                        const void* mask,
                        int64_t ldm, void* dx, int64_t lddx, void* du, int64_t lddu, float* dweight,
                        float* dbias, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Delta-q ("cached" / targets-only) attention: DS compact query rows per
 * sequence (delta_q [B*DS, H, D]) at positions L-DS .. L-1 of each sequence,
 * against that sequence's whole k / v [T, H, D] (L = min(length, N)), with
 * the _get_valid_attn_mask rows of those positions.  dtype is the k / v type
 * (bf16, or e4m3 with the per-tensor scales k_scale / v_scale), q_dtype the
 * delta q's (e4m3 with q_scale).  Output bf16 [B*DS, H, D]; D = 64 or 128.
 * Per-chunk fp32 partials go to the workspace and are summed in chunk order
 * (bitwise deterministic).
 * Replaces: triton_cached_hstu_mha, ops/triton/triton_hstu_attention.py:3710-3866
 *           (math of pytorch_cached_hstu_mha, ops/pytorch/pt_hstu_attention.py:191-251).
 */
int64_t hstu_delta_attn_workspace_bytes(int B, int H, int D, int N, int delta_size);
int hstu_delta_attn_fwd(int dtype, int q_dtype, const void* q, const void* k, const void* v,
                        int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                        float q_scale, float k_scale, float v_scale,
                        const int64_t* seq_offsets, int B, int H, int D, int max_seq_len, int delta_size,
                        float alpha, const int* num_targets, int max_attn_len, int contextual_seq_len,
                        void* out, int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                        hipStream_t stream);

/*
 * Backward of the delta attention (delta_size <= 4): writes dq [B*DS, H, D],
 * and dk, dv for every row of every sequence (zero where no delta query
 * attends, including rows past max_seq_len).  As in the reference, k and v
 * are dequantized and rounded to bf16 and silu / dS rounded to bf16 before use.
 * Replaces: triton_hstu_attention_delta_bwd, ops/triton/triton_hstu_attention.py:3413-3480
 *           (kernel _hstu_attn_delta_bwd :3033-3163).
 */
int hstu_delta_attn_bwd(int dtype, int q_dtype, const void* dout, int64_t dout_row_stride,
                        const void* q, const void* k, const void* v,
                        int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                        float q_scale, float k_scale, float v_scale,
                        const int64_t* seq_offsets, int B, int H, int D, int max_seq_len, int delta_size,
                        float alpha, const int* num_targets, int max_attn_len, int contextual_seq_len,
                        void* dq, void* dk, void* dv, int64_t dq_row_stride, int64_t dk_row_stride,
                        int64_t dv_row_stride, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * Block e4m3 quantization of the attention's upstream gradient (the input of
 * the full-FP8 backward): dout [T, H, D] bf16 (dtype HSTU_DTYPE_BF16) or fp32
 * (HSTU_DTYPE_FP32), row stride dout_row_stride elements, 16-byte aligned.
 * One power-of-two scale per (sequence, head, token group), the groups being
 * tokens p % 16 < 8 and p % 16 >= 8 of each 64-token tile of a sequence:
 * e = floor(log2(448 / amax)) from the fp32 bits, clamped to [-60, 60] (60 for
 * a subnormal amax, 0 for an all-zero group); dout_e4m3 [T, H, D] contiguous
 * = e4m3(dout * 2^e); e8 [T, H] uint8 = 127 - e.  Tiles cover the first
 * ceil(max_seq_len / 64) * 64 tokens of each sequence (max_seq_len >= every
 * length).  H * D in {128, 256, 512}, D in {64, 128}.
 * Replaces: quantize_do_e4m3_blk, ops/flydsl/hstu_do_fp8.py:95-121
 *           (kernel _blk_kernel :42-86, contract :16-38).
 */
int hstu_quantize_do_e4m3_blk(int dtype, const void* dout, int64_t dout_row_stride, const int64_t* seq_offsets,
                              int B, int H, int D, int max_seq_len, void* dout_e4m3, void* e8,
                              hipStream_t stream);

/*
 * The inverse, for a backward that runs on the block-quantized dO:
 * out[t, h, :] = bf16(dout_e4m3[t, h, :] * 2^(e8[t, h] - 127)), exact (an e4m3
 * value times a power of two within 2^+-60 is a bf16).  dout_e4m3 [T, H, D]
 * contiguous (8-byte aligned), e8 [T, H] uint8, out bf16 with row stride
 * out_row_stride elements (16-byte aligned rows); D % 8 == 0.
 * Replaces: the undoing of the block scales inside the full-FP8 backward's
 *           out-gemm MFMAs (ops/flydsl/hstu_flydsl_mha.py:1330-1394, do_blk).
 */
int hstu_dequantize_do_e4m3_blk(const void* dout_e4m3, const void* e8, int64_t T, int H, int D, void* out,
                                int64_t out_row_stride, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HSTU_MI355X_H_ */
