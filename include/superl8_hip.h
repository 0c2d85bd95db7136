/*
 * superl8_hip.h — C ABI of libsuperl8_hip.so, the gfx950 (MI355X) kernels
 * behind the superl8 INT8-attention / Q4_K-GEMV operator API.
 *
 * This library replaces the pybind11 module built from the reference's
 * csrc/fni8_api.cpp (superl8._C). Each entry point below names the reference
 * binding it stands in for. Conventions shared by every entry point:
 *
 *   - All tensor arguments are raw device pointers to contiguous row-major
 *     buffers, sizes are int64_t element counts, the stream is a hipStream_t
 *     passed as void* (NULL = the legacy default stream).
 *   - Outputs are allocated by the caller. Entry points never allocate,
 *     free or synchronise; work is enqueued on `stream` only.
 *   - Return value: SL8_OK (0) or a negative SL8_ERR_* code. The message for
 *     the last failure on the calling host thread is sl8_last_error().
 *     Argument checks mirror the reference's TORCH_CHECKs (same key phrases).
 *   - Scales are fp32. "Folded" Q scales carry softmax_scale*log2(e), so the
 *     kernels produce exp2-domain logits (reference superl8/quant/core.py:186-195).
 */
#ifndef SUPERL8_HIP_H
#define SUPERL8_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define SL8_OK 0
#define SL8_ERR_INVALID (-1) /* bad argument (shape, dtype, alignment, range) */
#define SL8_ERR_LAUNCH (-2)  /* HIP launch / runtime failure */

/* element types for dtype arguments */
#define SL8_DTYPE_F16 0
#define SL8_DTYPE_BF16 1
#define SL8_DTYPE_F32 2

/* Message of the last failed call on this host thread ("" if none). */
const char* sl8_last_error(void);

/* Library version string, e.g. "superl8-hip 0.1 gfx950". */
const char* sl8_version(void);

/* ------------------------------------------------------------------------
 * Per-row symmetric int8 quantisation.
 * Replaces _C.quantize_i8_rowwise (reference csrc/fni8_api.cpp:286-291,
 * csrc/kernel/quant_rowwise.cu:84-121, csrc/include/quant_rowwise.cuh:42-92).
 *   x [M,K] (x_dtype f16/bf16/f32) -> q int8 [M,K], scale fp32 [M]
 *   scale = amax|x_row| * fp32(1/127) (1 if 0); q = clamp(rint(x/scale), +-127)
 * ---------------------------------------------------------------------- */
int sl8_quantize_i8_rowwise(const void* x, int x_dtype, int64_t M, int64_t K,
                            int8_t* q, float* scale, void* stream);

/* ------------------------------------------------------------------------
 * K-smoothing mean: mean[g, d] = (1/N) * sum_n k[g, n, d], fp32.
 * Replaces the torch reduction in superl8/quant/core.py:29-44,70-95
 * (_mean_k_fp32_bounded / smooth_k). fp16 input is summed exactly in int64
 * fixed point (order-independent); bf16/f32 in fp64, rows in order.
 *   k [G, N, D] (dtype f16/bf16/f32) -> mean fp32 [G, D]
 * workspace: sl8_k_mean_workspace(G, D) bytes, 8-byte aligned (used for fp16:
 * the int64 partial sums; contents need not be initialised).
 * ---------------------------------------------------------------------- */
size_t sl8_k_mean_workspace(int64_t G, int64_t D);
int sl8_k_mean(const void* k, int dtype, int64_t G, int64_t N, int64_t D,
               float* mean, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Fused smooth + quantise (quantize_qk's K side, and Q with mean=NULL):
 *   xs[g,n,:] = dtype(x[g,n,:] - mean[g,:])      (mean may be NULL -> no shift)
 *   q, s      = per-row int8 of xs                 (as sl8_quantize_i8_rowwise)
 *   scale[g,n]= s * scale_mul                      (fp32 multiply; 1.0 = none)
 * Reference: superl8/quant/core.py:164-196 (smooth_k, quantize_int8_rowwise,
 * q_scale * (softmax_scale*LOG2E)).
 *   x [G, N, D] -> q int8 [G, N, D], scale fp32 [G, N]
 * ---------------------------------------------------------------------- */
int sl8_quantize_i8_rows_centered(const void* x, int x_dtype, int64_t G, int64_t N,
                                  int64_t D, const float* mean, float scale_mul,
                                  int8_t* q, float* scale, void* stream);

/* Row-group int8 quantisation: x [G][N][D] (f16/bf16/f32), one scale per
 * rows_per_group consecutive rows of each G slice (the last group of a slice
 * may be short): scale = amax over the group * fp32(1/127) (1 if zero),
 * codes and the optional mean shift as sl8_quantize_i8_rows_centered; every
 * row's entry of scale [G][N] holds its group's scale * scale_mul. The
 * per-wavefront Q / per-key-tile K quantisation of BASELINE config 5; no
 * counterpart in the reference (its Q/K scales are per row, core.py:164-196). */
int sl8_quantize_i8_row_groups(const void* x, int x_dtype, int64_t G, int64_t N, int64_t D,
                               int64_t rows_per_group, const float* mean, float scale_mul,
                               int8_t* q, float* scale, void* stream);

/* ------------------------------------------------------------------------
 * Fused fp16 attention prologue: quantize_qk (no rotation) plus, optionally,
 * the outlier gate, in two launches (six unfused). Replaces superl8/quant/core.py:164-196
 * (smooth_k + quantize_qk) and detect_q_outlier_domination (core.py:113-145)
 * as called from superl8/ops.py:115-150; results equal sl8_k_mean,
 * sl8_quantize_i8_rows_centered and sl8_q_outlier_gate bit for bit.
 *   q [qrows, D] fp16 (qrows = B*Hq*M), k [G, N, D] fp16 (G = B*Hkv), D in {64,128,256}
 *   -> q_i8 [qrows, D], q_scale [qrows] (x q_scale_mul), k_i8 [G, N, D],
 *      k_scale [G, N], k_mean fp32 [G, D]
 * gate_ratio > 0: *gate_flag = 1 if some Q row has max/(median+1e-10) > ratio,
 * else 0 (written, not OR-ed: no clearing needed). gate_ratio <= 0: no gate.
 * workspace: sl8_quantize_qk_workspace(qrows, G, N, D) bytes, 8-byte aligned,
 * uninitialised. q/k 16-byte aligned, codes 8-byte aligned; N < 2^23.
 * ---------------------------------------------------------------------- */
size_t sl8_quantize_qk_workspace(int64_t qrows, int64_t G, int64_t N, int64_t D);
int sl8_quantize_qk(const void* q, const void* k, int dtype, int64_t qrows, int64_t G, int64_t N,
                    int64_t D, float q_scale_mul, float gate_ratio, int8_t* q_i8, float* q_scale,
                    int8_t* k_i8, float* k_scale, float* k_mean, int32_t* gate_flag,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Per-channel int8 of V over the key axis (W8A8 path).
 * Replaces quantize_v_perchannel, reference superl8/quant/core.py:98-110
 * (on the GPU torch evaluates amax/127 as amax * fp32(1/127)).
 *   x [G, N, D] -> q int8 [G, N, D], scale fp32 [G, D]
 *   scale = amax_n|x| * fp32(1/127) (1 if 0); q = clamp(rint(x/scale), +-127)
 * ---------------------------------------------------------------------- */
int sl8_quantize_i8_cols(const void* x, int dtype, int64_t G, int64_t N, int64_t D, int8_t* q,
                         float* scale, void* stream);

/* ------------------------------------------------------------------------
 * Prefill FlashAttention-2: int8 QK^T on MFMA (int32 accumulate), fp32
 * online softmax in the exp2 domain, fp16/bf16 PV on MFMA, output dtype = V's.
 * Replaces _C.attn_int8_fwd / _C.attn_int8_fwd_train (reference
 * csrc/fni8_api.cpp:12-19,225-233, csrc/kernel/attn_int8_fwd.cu:101-200,
 * csrc/include/attn_int8_fwd.cuh:47-209).
 *   q int8 [B,Hq,M,D], q_scale fp32 [B,Hq,M] (folded), k int8 [B,Hkv,N,D],
 *   k_scale fp32 [B,Hkv,N], v [B,Hkv,N,D] (v_dtype f16/bf16),
 *   out [B,Hq,M,D] (v_dtype), lse fp32 [B,Hq,M] natural log or NULL.
 *   causal: bottom-right aligned (query i sees keys <= i + N - M).
 *   window_left >= 0: also require key > i + N - M - window_left.
 *   D in {32, 64, 72, 80, 128, 256} (reference attn_int8_fwd.cu:138). V is
 *   read in place; D = 32, 72, 80 run the 64- or 128-wide kernel on Q/K/V
 *   copies zero-padded in the workspace (sl8_attn_int8_fwd_workspace() bytes,
 *   0 for the other head dims).
 * ---------------------------------------------------------------------- */
size_t sl8_attn_int8_fwd_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N,
                                   int64_t D);
int sl8_attn_int8_fwd(const int8_t* q, const float* q_scale, const int8_t* k,
                      const float* k_scale, const void* v, int v_dtype, void* out,
                      float* lse, int64_t B, int64_t Hq, int64_t Hkv, int64_t M,
                      int64_t N, int64_t D, int causal, int64_t window_left,
                      void* workspace, size_t workspace_bytes, void* stream);

/* The same prefill for callers that decide an accuracy gate on the device:
 * when *gate_flag (device int32, written earlier on the same stream, e.g. by
 * sl8_quantize_qk) is nonzero every workgroup exits at once and out / lse are
 * left unwritten. No counterpart in the reference, which reads its gate on
 * the host before launching (superl8/ops.py:115-147); this lets the host read
 * the flag while the attention already runs. */
int sl8_attn_int8_fwd_gated(const int8_t* q, const float* q_scale, const int8_t* k,
                            const float* k_scale, const void* v, int v_dtype, void* out,
                            float* lse, int64_t B, int64_t Hq, int64_t Hkv, int64_t M,
                            int64_t N, int64_t D, int causal, int64_t window_left,
                            void* workspace, size_t workspace_bytes, const int32_t* gate_flag,
                            void* stream);

/* Test hook: the int32 Q.K^T scores exactly as the production prefill kernel
 * (sl8_attn_int8_fwd's attn_fwd_wide_kernel) computes them: the same template
 * instantiated with a dump epilogue, same tiling, pipeline and MFMA operands.
 *   scores int32 [B,Hq,M,N]; causal != 0 runs the causal kernel, which stores
 *   only the key tiles a wave computes (the caller pre-fills the rest).
 *   Head dims 32/72/80 need sl8_attn_int8_fwd_workspace() bytes of workspace.
 * No reference counterpart (the reference never exposes its dp4a
 * accumulators); used to prove bit-exact int32 QK^T. */
int sl8_attn_int8_qk_scores(const int8_t* q, const int8_t* k, int32_t* scores,
                            int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N,
                            int64_t D, int causal, void* workspace, size_t workspace_bytes,
                            void* stream);

/* ------------------------------------------------------------------------
 * Full W8A8 prefill: int8 QK^T and int8 PV (P re-quantised in-loop, per row
 * or per 32-key half), V int8 with per-channel scale, output fp16.
 * Replaces _C.attn_w8a8_fwd (reference csrc/fni8_api.cpp:30-33,249-255,
 * csrc/kernel/attn_w8a8_fwd.cu:76-165, csrc/include/attn_w8a8_fwd.cuh:30-444).
 *   v int8 [B,Hkv,N,D], v_scale fp32 [B,Hkv,D], causal_diag: query i sees
 *   keys <= i + causal_diag when causal. D in {32, 64, 128, 256} (reference
 *   attn_w8a8_fwd.cu:113; D = 32 runs zero-padded to 64 in the workspace).
 *   per_warp_quant: 0 = one P scale per 64-key tile (the reference's
 *   per_warp_quant=False); 1 = one P scale per 32-key half (the reference's
 *   default), P fed to the bf16 MFMA as code * 2^(max_half - m) / 127 (the
 *   rounding of that factor to bf16 is this build's only deviation); 2 = the
 *   same quantisation with the reference's exact arithmetic (int32 P.V per
 *   half, scaled in fp32), about twice the time of 1. No reference counterpart
 *   for 2 (the reference's per-warp path computes it this way).
 * ---------------------------------------------------------------------- */
size_t sl8_attn_w8a8_fwd_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t M, int64_t N,
                                   int64_t D);
int sl8_attn_w8a8_fwd(const int8_t* q, const float* q_scale, const int8_t* k,
                      const float* k_scale, const int8_t* v, const float* v_scale,
                      void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t M,
                      int64_t N, int64_t D, int causal, int64_t causal_diag,
                      int per_warp_quant, void* workspace, size_t workspace_bytes,
                      void* stream);

/* ------------------------------------------------------------------------
 * Split-KV decode (M = 1): int8 K with per-token fp32 scales, fp16 V,
 * per-split partials (O, m, l) merged by log-sum-exp, output fp16.
 * Replaces _C.attn_int8_decode (reference csrc/fni8_api.cpp:34-36,260-263,
 * csrc/kernel/attn_decode.cu:33-53,163-240, csrc/include/attn_decode.cuh:47-132,430-466).
 *   q int8 [B,Hq,1,D], q_scale fp32 [B,Hq] (folded), k int8 [B,Hkv,N,D],
 *   k_scale fp32 [B,Hkv,N], v fp16 [B,Hkv,N,D] -> out fp16 [B,Hq,1,D].
 *   num_splits: -1 = auto (sl8_choose_num_splits), else 1..256.
 *   D in {32, 64, 128, 256} (reference attn_decode.cu:195). workspace: sl8_attn_int8_decode_workspace() bytes.
 * ---------------------------------------------------------------------- */
int sl8_choose_num_splits(int64_t N, int64_t B, int64_t Hkv);
size_t sl8_attn_int8_decode_workspace(int64_t B, int64_t Hq, int64_t D, int64_t num_splits);
int sl8_attn_int8_decode(const int8_t* q, const float* q_scale, const int8_t* k,
                         const float* k_scale, const void* v, void* out, int64_t B,
                         int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                         int64_t num_splits, void* workspace, size_t workspace_bytes,
                         void* stream);

/* Split-KV decode with fp16 per-token K scales: k_scale_f16 [B,Hkv,N] (the
 * cache format of BASELINE config 3, half the scale bytes of the reference's
 * fp32 contract at csrc/kernel/attn_decode.cu:174-175). Otherwise exactly
 * sl8_attn_int8_decode (same workspace, checks and arithmetic after the
 * exact fp16 -> fp32 widening). Reached from _C.attn_int8_decode when
 * k_scale is float16. */
int sl8_attn_int8_decode_ks16(const int8_t* q, const float* q_scale, const int8_t* k,
                              const void* k_scale_f16, const void* v, void* out, int64_t B,
                              int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                              int64_t num_splits, void* workspace, size_t workspace_bytes,
                              void* stream);

/* Allocation-free split-KV decode. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc). Same arguments, checks,
 * kernels and results as sl8_attn_int8_decode, minus the workspace: the
 * per-split partials live in a static device array of
 * sl8_attn_int8_decode_noalloc_max_bytes() bytes (8 MiB) per device, looked up
 * on the first call on each device and held until the process ends. A call
 * whose partials (sl8_attn_int8_decode_workspace bytes) exceed it fails with
 * an error. Calls that overlap on one device share the array and race. Calls
 * no hipMalloc/hipFree. */
size_t sl8_attn_int8_decode_noalloc_max_bytes(void);
int sl8_attn_int8_decode_noalloc(const int8_t* q, const float* q_scale, const int8_t* k,
                                 const float* k_scale, const void* v, void* out, int64_t B,
                                 int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                                 int64_t num_splits, void* stream);

/* Split-KV decode over an int8 V cache: v int8 [B,Hkv,N,D] with per-channel
 * v_scale fp32 [B,Hkv,D], folded into each split's partial O. Otherwise as
 * sl8_attn_int8_decode (same workspace). Replaces _C.attn_int8_decode_kv8
 * (reference csrc/fni8_api.cpp:37-39,264-266, csrc/kernel/attn_decode.cu:100-118,242-320,
 * csrc/include/attn_decode.cuh:141-224). */
int sl8_attn_int8_decode_kv8(const int8_t* q, const float* q_scale, const int8_t* k,
                             const float* k_scale, const int8_t* v, const float* v_scale,
                             void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                             int64_t num_splits, void* workspace, size_t workspace_bytes,
                             void* stream);

/* Outlier gate of the prologue: *flag |= 1 when some row of q [rows, D]
 * (fp16/bf16/fp32, D in {64,128,256}) has max|q| / (median|q| + 1e-10) >
 * ratio in fp32, median = the lower middle element. flag must be zeroed by the
 * caller; stats, if not NULL, receives [rows][2] = (max, median). Replaces the
 * torch evaluation of detect_q_outlier_domination (reference
 * superl8/quant/core.py:113-145, called by superl8/ops.py:115-147). */
int sl8_q_outlier_gate(const void* q, int dtype, int64_t rows, int64_t D, float ratio,
                       int32_t* flag, float* stats, void* stream);

/* ------------------------------------------------------------------------
 * Paged int8 KV cache (reference csrc/fni8_api.cpp:138-143,152-154,509-527,
 * csrc/kernel/attn_paged_decode.cu:14-31,107-240,360-421,
 * csrc/include/attn_paged_decode.cuh:55-262).
 *   k_cache, v_cache int8 [num_blocks, Hkv, block_size, D]; k_scale, v_scale
 *   fp32 [num_blocks, Hkv, block_size] (per token). block_table int32
 *   [B, max_blocks_per_seq]: physical block of each logical block of a
 *   sequence; context_lens int32 [B]. Splits are sized on max_context_len
 *   (<= max_blocks_per_seq * block_size); num_splits -1 = auto
 *   (sl8_paged_choose_num_splits). Workspace: sl8_attn_int8_decode_workspace.
 * sl8_kv_write_paged: quantise one new token per (batch, KV head) from fp16
 *   k_new, v_new [B, Hkv, D] into flat slot_mapping[b] = block*bs + offset,
 *   in place (scale = amax / 127, code = rint(x / scale)).
 * ---------------------------------------------------------------------- */
int sl8_paged_choose_num_splits(int64_t n_len_max, int64_t bhq);
int sl8_attn_paged_decode(const int8_t* q, const float* q_scale, const int8_t* k_cache,
                          const float* k_scale, const int8_t* v_cache, const float* v_scale,
                          const int32_t* block_table, const int32_t* context_lens, void* out,
                          int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t num_blocks,
                          int64_t block_size, int64_t max_blocks_per_seq,
                          int64_t max_context_len, int64_t num_splits, void* workspace,
                          size_t workspace_bytes, void* stream);
/* K8V3 paged decode: replaces _C.attn_paged_decode_k8v3 (reference
 * csrc/fni8_api.cpp:144-151,516-519, csrc/kernel/attn_paged_decode.cu:67-89,229-330,
 * csrc/include/attn_paged_decode.cuh:134-257 with LowbitV). K, scales, block
 * table, context lengths, splits and workspace as sl8_attn_paged_decode; V is
 * the 3-bit Lloyd-Max store: v_packed int32 [num_blocks, Hkv, block_size, 3D/32]
 * (code of channel d at bits 3d..3d+2 of the row's LSB-first stream), v_norm
 * fp32 [num_blocks, Hkv, block_size, D/128] (per-128-channel L2 norms),
 * v_codebook fp32 [8]; value = fp16_rn(codebook[code] * norm). D 128 or 256;
 * k_cache and v_packed 16-byte aligned. */
int sl8_attn_paged_decode_k8v3(const int8_t* q, const float* q_scale, const int8_t* k_cache,
                               const float* k_scale, const int32_t* v_packed,
                               const float* v_norm, const float* v_codebook,
                               const int32_t* block_table, const int32_t* context_lens,
                               void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                               int64_t num_blocks, int64_t block_size,
                               int64_t max_blocks_per_seq, int64_t max_context_len,
                               int64_t num_splits, void* workspace, size_t workspace_bytes,
                               void* stream);
int sl8_kv_write_paged(const void* k_new, const void* v_new, const int32_t* slot_mapping,
                       int8_t* k_cache, float* k_scale, int8_t* v_cache, float* v_scale,
                       int64_t B, int64_t Hkv, int64_t D, int64_t num_blocks,
                       int64_t block_size, void* stream);

/* ------------------------------------------------------------------------
 * Q4_K GEMM/GEMV over native GGUF super-blocks (144 B per 256 weights:
 * fp16 d, fp16 dmin, 12 B packed 6-bit sub-scales/mins, 128 B nibbles).
 *   y[m,n] = x_scale[m] * sum_j (d*sc_j*<x_j,q_j> - dmin*m_j*sum(x_j))
 *   x int8 [M,K] (K % 256 == 0), x_scale fp32 [M], w uint8 [N, K/256*144],
 *   out [M,N] out_dtype (f16 / bf16 as the reference; f32 also accepted).
 * sl8_gemm_decode_q4k replaces _C.gemm_decode_q4k (reference
 * csrc/fni8_api.cpp:346-352, csrc/kernel/gemm_decode_dp4a.cu:375-436,
 * csrc/include/gemm_decode_dp4a.cuh:476-537); M <= 16.
 * sl8_gemm_q4k replaces _C.gemm_q4k (reference csrc/fni8_api.cpp:331-337,
 * csrc/kernel/gemm_dp4a.cu:146-193, csrc/include/gemm_q4k_dp4a.cuh:60-199); any M.
 * ---------------------------------------------------------------------- */
int sl8_gemm_decode_q4k(const int8_t* x, const float* x_scale, const uint8_t* w,
                        void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                        void* stream);

/* Decode GEMV with per-256-block activation scales: x_scale [M, K/256] fp32
 * (one scale per super-block-aligned slice of each activation row, the
 * activation format of BASELINE config 4) multiplies each super-block's
 * exact integer sums. No counterpart in the reference, whose activations
 * carry one scale per row (csrc/kernel/gemm_decode_dp4a.cu:398); otherwise as
 * sl8_gemm_decode_q4k (M <= 16, same checks). */
int sl8_gemm_decode_q4k_xblock(const int8_t* x, const float* x_scale, const uint8_t* w,
                               void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                               void* stream);
int sl8_gemm_q4k(const int8_t* x, const float* x_scale, const uint8_t* w, void* out,
                 int out_dtype, int64_t M, int64_t N, int64_t K, void* stream);

/* Dequantise native Q4_K bytes to fp32 [N,K]: w = fp32(d)*sc*q - fp32(dmin)*m
 * (exact in fp32). Reference math: csrc/include/gemm_q4k_dp4a.cuh:35-51 and
 * the test decoder tests/test_gemm_q4k.py:132-148. */
int sl8_dequant_q4k(const uint8_t* w, float* out, int64_t N, int64_t K, void* stream);

/* ------------------------------------------------------------------------
 * GGUF Q5_K / Q6_K linear (native 176 / 210-byte super-blocks), same
 * arguments and contract as the Q4_K pair above:
 *   Q5_K: y = x_scale * sum_j (d*sc_j*<x_j,q_j> - dmin*m_j*sum(x_j)), q 5-bit
 *   Q6_K: y = x_scale * sum_i d*sc_i*<x_i, q_i - 32>, 16-element sub-blocks
 * sl8_gemm_q5k / sl8_gemm_q6k replace _C.gemm_q5k / _C.gemm_q6k (reference
 * csrc/fni8_api.cpp:64-67,338-347, csrc/include/gemm_q4k_dp4a.cuh:200-489); any M.
 * sl8_gemm_decode_q5k / _q6k replace _C.gemm_decode_q5k / _q6k (fni8_api.cpp:
 * 70-73,353-360, csrc/kernel/gemm_decode_dp4a.cu:377-446); M <= 16.
 * The Q6_K weight buffer is read in whole dwords: it must stay readable up to
 * its end rounded up to 4 bytes (torch allocations always are).
 * sl8_dequant_q5k / _q6k: bytes -> fp32 [N, K], as the reference test decoders
 * (tests/test_gemm_q4k.py:188-190,218-221). */
int sl8_gemm_q5k(const int8_t* x, const float* x_scale, const uint8_t* w, void* out,
                 int out_dtype, int64_t M, int64_t N, int64_t K, void* stream);
int sl8_gemm_q6k(const int8_t* x, const float* x_scale, const uint8_t* w, void* out,
                 int out_dtype, int64_t M, int64_t N, int64_t K, void* stream);
int sl8_gemm_decode_q5k(const int8_t* x, const float* x_scale, const uint8_t* w, void* out,
                        int out_dtype, int64_t M, int64_t N, int64_t K, void* stream);
int sl8_gemm_decode_q6k(const int8_t* x, const float* x_scale, const uint8_t* w, void* out,
                        int out_dtype, int64_t M, int64_t N, int64_t K, void* stream);
int sl8_dequant_q5k(const uint8_t* w, float* out, int64_t N, int64_t K, void* stream);
int sl8_dequant_q6k(const uint8_t* w, float* out, int64_t N, int64_t K, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SUPERL8_HIP_H */
