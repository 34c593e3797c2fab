/*
 * StreamIndex for MI355X — C ABI of libstreamindex.so.
 *
 * Plain pointers, element strides and sizes; no torch or HIP C++ types.  All
 * device pointers are HIP device memory; `stream` is a hipStream_t passed as
 * void* (NULL = the default stream).  Every call is asynchronous on `stream`,
 * allocates nothing, and returns a status code:
 *
 *   0 SI_OK, 1 SI_ERR_INVALID (bad argument), 2 SI_ERR_UNSUPPORTED (valid but
 *   outside the implemented shapes), 3 SI_ERR_LAUNCH (HIP launch error).
 *
 * On a non-zero status si_last_error() returns a thread-local description.
 *
 * The reference (tsukimia-hoshi/StreamIndex) is Python + Triton with no C
 * FFI; each entry below replaces one of its Python operators, cited by
 * file:line in the reference tree.  The Python binding that mirrors those
 * operators is streamindex_amd/_lib.py (ctypes).
 */
#ifndef STREAMINDEX_H_
#define STREAMINDEX_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SI_OK 0
#define SI_ERR_INVALID 1
#define SI_ERR_UNSUPPORTED 2
#define SI_ERR_LAUNCH 3

/* Element type of the sparse-attention operands q, kv, o (and dO, dq, dkv). */
#define SI_DTYPE_BF16 0
#define SI_DTYPE_F16 1

/* Version of this interface (incremented on any signature change). */
int si_abi_version(void);

/* Thread-local text of the last error returned on this thread. */
const char* si_last_error(void);

/*
 * Device workspace si_indexer_topk needs (always 0: selection state lives in
 * LDS).  Replaces the chunk_s x chunk_t fp32 score tile the reference driver
 * allocates per (s-chunk, t-chunk) pair,
 * flash_sparse/triton/chunked_indexer.py:92-118.
 */
size_t si_indexer_topk_workspace_bytes(int64_t B, int64_t S, int64_t T, int64_t H, int64_t D,
                                       int64_t top_k);

/*
 * Fused lightning-indexer score + exact top-k per query row.
 * Replaces flash_sparse/triton/chunked_indexer.py:47-160 (chunked_indexer_topk)
 * and, with out width min(top_k,T), indexer_score.py:182-205 (indexer_score_topk).
 *
 *   q        [B,S,H,D] bf16, strides q_strides[4] (elements; last must be 1)
 *   k_idx    [B,T,D]   bf16, strides k_strides[3] (last must be 1)
 *   weights  [B,S,H]   fp32 (w_dtype 0) or bf16 (w_dtype 1), strides w_strides[3]
 *   mask     optional [B,S,T] bool (1 byte, nonzero = legal), strides mask_strides[3]; NULL = none
 *   causal_ratio > 0: key t legal for row s iff t < (s+1)/causal_ratio; 0 = none.
 *                     Must be 0 when mask != NULL.
 *   out_idx    [B,S,top_k] int64, contiguous: best-first, -1 past the legal count
 *   out_scores [B,S,top_k] fp32,  contiguous: best-first, -inf past the legal count
 * Ties rank the smaller key index first.  Supported: D in {32,64,128,256},
 * 1 <= H <= 256, 1 <= top_k <= 4096 (the reference takes any power-of-two
 * H >= 16 and D, flash_sparse/triton/indexer_score.py:145-150, and any
 * top_k, chunked_indexer.py:47-57).
 */
int si_indexer_topk(const void* q, const int64_t* q_strides, const void* k_idx, const int64_t* k_strides,
                    const void* weights, int w_dtype, const int64_t* w_strides, const uint8_t* mask,
                    const int64_t* mask_strides, int64_t B, int64_t S, int64_t T, int64_t H, int64_t D,
                    int64_t top_k, int64_t causal_ratio, int64_t* out_idx, float* out_scores, void* stream);

/*
 * Which top-k kernel si_indexer_topk and si_csa_indexer_topk launch
 * (process-wide; returns the previous setting).  No counterpart in the
 * reference: a tuning and test knob.  SI_TOPK_KERNEL_AUTO (default) runs
 * the four-32-head-block kernel for D = 128 with H in (96, 128], or H in
 * (32, 64] and rows of at least 64K legal keys, and the
 * two-workgroups-per-CU kernel otherwise; _NARROW and _WIDE force one of
 * them where the shape allows (WIDE falls back to NARROW for the shapes
 * only NARROW serves, e.g. top_k > 1152 at H <= 64).  Both return
 * identical results.  Returns the previous mode, or -1 for a mode
 * outside 0..2.
 */
#define SI_TOPK_KERNEL_AUTO 0
#define SI_TOPK_KERNEL_NARROW 1
#define SI_TOPK_KERNEL_WIDE 2
int si_indexer_set_topk_kernel(int mode);

/*
 * The kernel si_indexer_topk would launch for a shape under the current
 * si_indexer_set_topk_kernel mode, without launching anything.  *kernel
 * receives 1 (one query row per wave, two workgroups per CU where registers
 * allow: H <= 128, or 64 at D = 256, and top_k <= 2048, or 1536 at D = 256),
 * 2 (four 32-head blocks per wave: D = 128, T >= 64, top_k <= 1152) or 3
 * (each row's heads split over two or four waves: the other shapes up to
 * H = 256 and top_k = 4096); *capacity the selection buffer's keys per row.
 * Either pointer may be NULL.  Returns a status code (SI_ERR_UNSUPPORTED
 * for a shape no kernel serves).  No counterpart in the reference: a
 * planning query for tests and tuning.
 */
int si_indexer_topk_plan(int64_t S, int64_t T, int64_t H, int64_t D, int64_t top_k, int64_t causal_ratio,
                         int32_t* kernel, int32_t* capacity);

/*
 * Materialised indexer score matrix scores[b,s,t] = sum_h w[b,s,h]*relu(q[b,s,h,:].k[b,t,:]),
 * fp32 with strides score_strides[3].  No mask.
 * Replaces flash_sparse/triton/indexer_score.py:41-179 (_indexer_score_kernel, indexer_score).
 */
int si_indexer_score(const void* q, const int64_t* q_strides, const void* k_idx, const int64_t* k_strides,
                     const void* weights, int w_dtype, const int64_t* w_strides, int64_t B, int64_t S,
                     int64_t T, int64_t H, int64_t D, float* scores, const int64_t* score_strides,
                     void* stream);

/*
 * MQA sparse attention forward with attention sink.
 * Replaces flash_sparse/triton/sparse_attn_fwd.py:40-292 (_sparse_attn_fwd_kernel, sparse_attn_fwd).
 *
 *   q [B,S,H,D] and kv [B,N_kv,D] of one element type, qkv_dtype SI_DTYPE_BF16 or
 *   SI_DTYPE_F16 (sparse_attn_fwd.py:193,207 accept both); attn_sink [H] fp32;
 *   topk_idxs [B,S,K] int32 (idx_is_i64 = 0) or int64 (1); -1 or >= N_kv = masked.
 *   o [B,S,H,D] out, q's type; lse [B,S,H] fp32 out (natural log, sink included).
 *   P is rounded to the element type before P.V, as the reference does.
 * Supported: any H (64-head groups), D in {32,64,128,256,512,576}.
 */
int si_sparse_attn_fwd(const void* q, const int64_t* q_strides, const void* kv, const int64_t* kv_strides,
                       const float* attn_sink, const void* topk_idxs, int idx_is_i64,
                       const int64_t* idx_strides, int64_t B, int64_t S, int64_t H, int64_t D, int64_t N_kv,
                       int64_t K, float softmax_scale, int qkv_dtype, void* o, const int64_t* o_strides, float* lse,
                       const int64_t* lse_strides, void* stream);

/*
 * si_sparse_attn_fwd with optional per-row column counts: row_len [B,S]
 * int32 (strides in elements); columns j >= row_len[b,s] are masked and the
 * 32-key tiles past it are never gathered or computed.  row_len = NULL is
 * si_sparse_attn_fwd.  No counterpart in the reference (whose HCA rows,
 * flash_sparse/hca.py:40-51, carry a -1 tail of known length through
 * sparse_attn_fwd.py:180-292); used by the HCA / CSA compositions.
 */
int si_sparse_attn_fwd_ragged(const void* q, const int64_t* q_strides, const void* kv, const int64_t* kv_strides,
                              const float* attn_sink, const void* topk_idxs, int idx_is_i64,
                              const int64_t* idx_strides, int64_t B, int64_t S, int64_t H, int64_t D, int64_t N_kv,
                              int64_t K, float softmax_scale, int qkv_dtype, void* o, const int64_t* o_strides, float* lse,
                              const int64_t* lse_strides, const int32_t* row_len, const int64_t* row_len_strides,
                              void* stream);

/*
 * si_sparse_attn_fwd_ragged over two KV tensors read in place: indices in
 * [0, N_kv) select rows of kv [B,N_kv,D], indices in [N_kv, N_kv + N_kv2)
 * rows of kv2 [B,N_kv2,D] (same element type, strides kv2_strides[3]).
 * Equal to si_sparse_attn_fwd_ragged over their concatenation along N.
 * topk_idxs is int32; N_kv + N_kv2 must fit in int32.  Replaces
 * the torch.cat([kv, kv_compressed]) that feeds sparse_attn_fwd in
 * flash_sparse/csa.py:197-205 and flash_sparse/hca.py:85-95.
 */
int si_sparse_attn_fwd_kv2(const void* q, const int64_t* q_strides, const void* kv, const int64_t* kv_strides,
                           int64_t N_kv, const void* kv2, const int64_t* kv2_strides, int64_t N_kv2,
                           const float* attn_sink, const int32_t* topk_idxs, const int64_t* idx_strides, int64_t B,
                           int64_t S, int64_t H, int64_t D, int64_t K, float softmax_scale, int qkv_dtype, void* o,
                           const int64_t* o_strides, float* lse, const int64_t* lse_strides, const int32_t* row_len,
                           const int64_t* row_len_strides, void* stream);

/*
 * Fused indexer top-k that writes CSA attention index rows directly.
 * Replaces flash_sparse/csa.py:149-179 (chunked indexer, window indices,
 * "+S" offset of the compressed picks, int32 concat) and, for the same
 * result without the [B,S,T] score matrix, csa.py:181-196 (indexer_score +
 * build_csa_topk_idxs).
 *
 *   q, k_idx, weights, B..D, top_k, causal_ratio: as si_indexer_topk (no mask).
 *   out_idx [B,S,n_win+top_k] int32, strides out_strides[3] (last must be 1):
 *     column j < n_win: s - n_win + 1 + j, or -1 where negative;
 *     column n_win + r: the r-th best legal key + idx_offset, -1 past the legal count.
 *   out_scores: optional [B,S,top_k] fp32 contiguous (NULL = not written).
 * Needs idx_offset + T < 2^31.
 */
int si_csa_indexer_topk(const void* q, const int64_t* q_strides, const void* k_idx, const int64_t* k_strides,
                        const void* weights, int w_dtype, const int64_t* w_strides, int64_t B, int64_t S,
                        int64_t T, int64_t H, int64_t D, int64_t top_k, int64_t causal_ratio, int64_t n_win,
                        int64_t idx_offset, int32_t* out_idx, const int64_t* out_strides, float* out_scores,
                        void* stream);

/*
 * CSA attention index rows from a materialised score matrix.
 * Replaces flash_sparse/csa.py:30-83 (build_csa_topk_idxs).
 *
 *   scores [B,S,T] fp32 with strides score_strides[3]; key t legal for row s iff
 *   t < (s+1)/causal_ratio (causal_ratio 0: all legal) and its score is not -inf.
 *   out_idx: as si_csa_indexer_topk.  Ties rank the smaller index first.
 *   Supported: 1 <= top_k <= 2048.
 */
int si_csa_scores_topk(const float* scores, const int64_t* score_strides, int64_t B, int64_t S, int64_t T,
                       int64_t top_k, int64_t causal_ratio, int64_t n_win, int64_t idx_offset, int32_t* out_idx,
                       const int64_t* out_strides, void* stream);

/*
 * HCA attention index rows: window columns as above, then column n_win + i =
 * i + idx_offset if m_prime*(i+1) - 1 <= s, else -1, for i < n_compressed.
 * Replaces flash_sparse/hca.py:24-51 (build_hca_topk_idxs).
 *   out_idx [B,S,n_win+n_compressed] int32, strides out_strides[3] (last must be 1).
 */
int si_hca_topk_idxs(int64_t B, int64_t S, int64_t n_win, int64_t n_compressed, int64_t m_prime,
                     int64_t idx_offset, int32_t* out_idx, const int64_t* out_strides, void* stream);

/*
 * Workspace of si_sparse_attn_bwd: the bytes needed to process the query
 * rows in the fewest chunks that fit max_bytes (one chunk when the whole
 * problem fits), or, when even one row does not fit, the one-row need.
 * Returns -1 on bad arguments (si_last_error() says why).
 */
int64_t si_sparse_attn_bwd_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t D, int64_t N_kv, int64_t K,
                                           int64_t max_bytes);

/*
 * Sparse-attention backward from the forward's saved o and lse.
 * Replaces flash_sparse/triton/sparse_attn_bwd.py:286-416 (sparse_attn_bwd:
 * _delta_kernel + _sparse_attn_bwd_kernel) and is what the autograd wrapper
 * flash_sparse/triton/__init__.py:37-44 calls.
 *
 *   q, kv, attn_sink, topk_idxs, B..K, softmax_scale: as si_sparse_attn_fwd.
 *   o [B,S,H,D] bf16, lse [B,S,H] fp32: the forward's outputs; dout: dL/do.
 *   dq [B,S,H,D] bf16 (written), dkv [B,N_kv,D] bf16 (written; rows no query
 *   selects are 0), dsink [H] fp32 (written).
 *   workspace: at least si_sparse_attn_bwd_workspace_bytes(..., workspace_bytes)
 *   bytes, 16-byte aligned; the rows are processed in chunks that fit it.
 * dkv is reduced key by key in a fixed order (no atomics): repeated calls
 * give identical results.  Supported: H <= 128, D in {32,64,128,256,512,576},
 * B*S < 2^31, B*N_kv < 2^31.
 */
int si_sparse_attn_bwd(const void* q, const int64_t* q_strides, const void* kv, const int64_t* kv_strides,
                       const float* attn_sink, const void* topk_idxs, int idx_is_i64, const int64_t* idx_strides,
                       const void* o, const int64_t* o_strides, const float* lse, const int64_t* lse_strides,
                       const void* dout, const int64_t* do_strides, int64_t B, int64_t S, int64_t H, int64_t D,
                       int64_t N_kv, int64_t K, float softmax_scale, int qkv_dtype, void* dq, const int64_t* dq_strides, void* dkv,
                       const int64_t* dkv_strides, float* dsink, void* workspace, int64_t workspace_bytes,
                       void* stream);

/*
 * si_sparse_attn_bwd with optional per-row column counts, as
 * si_sparse_attn_fwd_ragged: row_len [B,S] int32 (strides in elements);
 * columns j >= row_len[b,s] are masked and their tiles are skipped.  No
 * counterpart in the reference; the backward of the HCA / CSA compositions.
 * The workspace is sized as for si_sparse_attn_bwd.
 */
int si_sparse_attn_bwd_ragged(const void* q, const int64_t* q_strides, const void* kv, const int64_t* kv_strides,
                              const float* attn_sink, const void* topk_idxs, int idx_is_i64,
                              const int64_t* idx_strides, const void* o, const int64_t* o_strides, const float* lse,
                              const int64_t* lse_strides, const void* dout, const int64_t* do_strides, int64_t B,
                              int64_t S, int64_t H, int64_t D, int64_t N_kv, int64_t K, float softmax_scale, int qkv_dtype, void* dq,
                              const int64_t* dq_strides, void* dkv, const int64_t* dkv_strides, float* dsink,
                              void* workspace, int64_t workspace_bytes, const int32_t* row_len,
                              const int64_t* row_len_strides, void* stream);

/*
 * si_sparse_attn_bwd_ragged without allocation: the workspace is a
 * file-scope device array of si_sparse_attn_bwd_noalloc_scratch_bytes()
 * bytes (128 MiB) that each GPU holds from library load until the process
 * ends; nothing is allocated and no workspace argument is taken.  No
 * counterpart in the reference: for callers that cannot allocate device
 * memory (HIP graph capture, tight training loops, harnesses that forbid
 * hipMalloc).  Arguments and results as si_sparse_attn_bwd_ragged.  Rows are
 * processed in chunks that fit the scratch; a problem whose smallest plan
 * (one query row per chunk: 4*B*S*64*ceil(H/64) + 8*B*N_kv + 4*B*N_kv*D bytes
 * plus one row's coefficients, per-slot rows and sort buffers) exceeds it is
 * rejected with SI_ERR_UNSUPPORTED before any launch.  All calls on one GPU
 * share that GPU's array: calls that overlap on one GPU (other threads or
 * streams) race.
 */
int64_t si_sparse_attn_bwd_noalloc_scratch_bytes(void);
int si_sparse_attn_bwd_noalloc(const void* q, const int64_t* q_strides, const void* kv, const int64_t* kv_strides,
                               const float* attn_sink, const void* topk_idxs, int idx_is_i64,
                               const int64_t* idx_strides, const void* o, const int64_t* o_strides, const float* lse,
                               const int64_t* lse_strides, const void* dout, const int64_t* do_strides, int64_t B,
                               int64_t S, int64_t H, int64_t D, int64_t N_kv, int64_t K, float softmax_scale, int qkv_dtype, void* dq,
                               const int64_t* dq_strides, void* dkv, const int64_t* dkv_strides, float* dsink,
                               const int32_t* row_len, const int64_t* row_len_strides, void* stream);

/*
 * Inverted top-k index.  Replaces flash_sparse/triton/inverted_topk.py:75-128
 * (build_inverted_topk).
 *   topk_idxs [B,S,K] int32 / int64 (strides in elements); keys outside [0, n_kv) ignored.
 *   inv_count [B,n_kv] int32: pairs selecting each key (not clamped);
 *   inv_topk [B,n_kv,k_max] int32: their query indices in ascending (query, slot)
 *   order, -1 past min(count, k_max).
 *   workspace: si_build_inverted_topk_workspace_bytes(B, S, K, n_kv) bytes.
 */
int64_t si_build_inverted_topk_workspace_bytes(int64_t B, int64_t S, int64_t K, int64_t n_kv);
int si_build_inverted_topk(const void* topk_idxs, int idx_is_i64, const int64_t* idx_strides, int64_t B, int64_t S,
                           int64_t K, int64_t n_kv, int64_t k_max, int32_t* inv_topk, int32_t* inv_count,
                           void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Indexer + exact top-k over quantised inputs (the production V4 indexer
 * dtypes: fp4 queries, fp8 keys).  Same operator as si_indexer_topk
 * (flash_sparse/triton/chunked_indexer.py:47-160) on the dequantised values
 * q = e2m1 * q_scale, k = e4m3 * k_scale.
 *   q_fp4 [B,S,H,D/2] uint8 (element 2i in the low nibble), byte strides q_strides[4];
 *   q_scale [B,S,H,D/32] fp32 powers of two (their exponent bits are used as UE8M0);
 *   k_fp8 [B,T,D] e4m3 bytes, byte strides k_strides[3]; k_scale [B,T] fp32 > 0;
 *   weights, causal_mask, causal_ratio, outputs: as si_indexer_topk.
 * Supported: H <= 64, D = 128, 1 <= top_k <= 2048; byte strides multiples of 16.
 */
int si_indexer_topk_q(const void* q_fp4, const int64_t* q_strides, const float* q_scale,
                      const int64_t* q_scale_strides, const void* k_fp8, const int64_t* k_strides,
                      const float* k_scale, const int64_t* k_scale_strides, const void* weights, int w_dtype,
                      const int64_t* w_strides, const uint8_t* causal_mask, const int64_t* mask_strides, int64_t B,
                      int64_t S, int64_t T, int64_t H, int64_t D, int64_t top_k, int64_t causal_ratio,
                      int64_t* out_idx, float* out_scores, void* stream);

/*
 * si_indexer_topk_q writing CSA attention index rows, as si_csa_indexer_topk
 * does for bf16 inputs (window columns, then the picks + idx_offset, -1 past
 * the legal count).  Replaces flash_sparse/csa.py:149-179 under the
 * production indexer dtypes.
 */
int si_csa_indexer_topk_q(const void* q_fp4, const int64_t* q_strides, const float* q_scale,
                          const int64_t* q_scale_strides, const void* k_fp8, const int64_t* k_strides,
                          const float* k_scale, const int64_t* k_scale_strides, const void* weights, int w_dtype,
                          const int64_t* w_strides, int64_t B, int64_t S, int64_t T, int64_t H, int64_t D,
                          int64_t top_k, int64_t causal_ratio, int64_t n_win, int64_t idx_offset, int32_t* out_idx,
                          const int64_t* out_strides, float* out_scores, void* stream);

/*
 * Block quantise-dequantise simulations, bit-identical to the reference formulas.
 * Replaces flash_sparse/utils/quantization.py:19-37 (fp4 = 0: act_quant_simulate,
 * fp8 e4m3, scale = amax / 448) and :40-65 (fp4 = 1: fp4_act_quant_simulate,
 * e2m1 grid, scale = amax / 6).
 *   x, y: n contiguous elements of dtype 0 = fp32, 1 = bf16, 2 = fp16; blocks of
 *   block_size consecutive elements (block_size = 8 * 2^j <= 512, n % block_size == 0).
 */
int si_quant_simulate(const void* x, void* y, int dtype, int64_t n, int64_t block_size, int fp4, void* stream);

/*
 * Packed production formats named by flash_sparse/utils/quantization.py:3-9
 * (DeepSeek-V4 act_quant / fp4_act_quant).
 *   fp4 = 0: y = n fp8 e4m3 bytes, scale[n / block_size] fp32 = max(amax, 1e-4) / 448
 *            (pow2_scale: rounded up to a power of two, UE8M0);
 *   fp4 = 1: y = n / 2 bytes of e2m1 pairs (element 2i in the low nibble),
 *            scale = power of two >= max(amax, 6 * 2^-126) / 6.
 *   Values are rounded to nearest, ties to even.
 */
int si_quant_pack(const void* x, void* y, float* scale, int dtype, int64_t n, int64_t block_size, int fp4,
                  int pow2_scale, void* stream);

/*
 * Token compressor (softmax-gated pooling of m tokens into one entry).
 * Replaces flash_sparse/reference.py:176-272 (reference_token_compressor).
 *   c_a, z_a [B,S,C] (dtype as above), b_a [m,C] fp32; overlap = 1 (CSA, eq. 11-12)
 *   also c_b, z_b [B,S,C] and b_b [m,C]: entry i pools block i of stream a and
 *   block i-1 of stream b (none for i = 0).  out [B, S/m, C] (trailing tokens dropped).
 */
int si_token_compress(const void* c_a, const void* z_a, const float* b_a, const void* c_b, const void* z_b,
                      const float* b_b, int dtype, int64_t B, int64_t S, int64_t C, int64_t m, int overlap, void* out,
                      void* stream);

/*
 * out[o, i] = sum_l kv[o, l, i] softmax_l(score[o, :, i]) over contiguous [outer, L, inner].
 * Replaces flash_sparse/utils/compression.py:13-24 (softmax_gated_pool).
 */
int si_gated_pool(const void* kv, const void* score, void* out, int dtype, int64_t outer, int64_t L, int64_t inner,
                  void* stream);

/*
 * Synthetic inputs for benchmarks and tests (no counterpart in the reference,
 * whose harnesses draw with torch.randn on a CUDA generator,
 * eval/test_v4_indexer_parity.py:89-103): out[i] = N(0,1)[seed, stream, i]
 * * scale, i < n, as fp32 (dtype 0) or bf16 rounded to nearest even (dtype 1).
 * Element i depends on (seed, stream, i) only (Philox4x32-10 counter (i/4,
 * stream, 0), Box-Muller with IEEE-exact ln / sin / cos polynomials), so the
 * same tensor results on every device and launch shape and any slice can be
 * recomputed on the CPU.
 */
int si_fill_normal(void* out, int dtype, int64_t n, uint64_t seed, uint32_t stream, float scale, void* stream_ptr);

#ifdef __cplusplus
}
#endif

#endif /* STREAMINDEX_H_ */
