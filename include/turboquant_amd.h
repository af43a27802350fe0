/*
 * turboquant_amd.h -- C ABI of the MI355X (gfx950) TurboQuant quantized
 * paged-KV hot path.  Plain pointers and sizes only; every device pointer is
 * HIP device memory owned by the caller, every launch goes on `stream`, no
 * call allocates or synchronises.
 *
 * Cache layout (fixed by the vLLM page-size hook of the reference,
 * turboquant/vllm_backend_fused.py:56-86):
 *   kv_cache uint8 [2, num_blocks, block_size, num_kv_heads, ebs]
 *   pd = next_pow2(head_dim) in {64,128,256}, qbytes = pd/2,
 *   ebs = (qbytes + 2*(pd/64) + 15) & ~15  (48 / 80 / 144 bytes)
 *   entry bytes [0, qbytes): 4-bit codes, dim 2k in the high nibble of byte k
 *   entry bytes [qbytes, qbytes + 2*pd/64): fp16 norm repeated pd/64 times
 *   the K slab is kv_cache[0], the V slab kv_cache[1].
 *
 * Return value: 0 on success, -22 (-EINVAL) for bad arguments, otherwise the
 * hipError_t of the launch.  tq_last_error() returns a message for the last
 * non-zero return on the calling thread.
 */
#ifndef TURBOQUANT_AMD_H
#define TURBOQUANT_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* tq_stream_t; /* == hipStream_t */

enum tq_dtype { TQ_F32 = 0, TQ_F16 = 1, TQ_BF16 = 2 };

/*
 * Quantize K and V rows and scatter them into the paged cache.
 *
 * Replaces turboquant_write::quantize_write_kv_cache
 * (reference csrc/src/quantize_write_binding.cu:207-269, kernel
 * csrc/include/turboquant/quantize_write_kernel.cuh:332-431), which the
 * backend calls from TurboQuantFusedImpl._write_to_cache
 * (turboquant/vllm_backend_fused.py:293-305).
 *
 * key/value: element (t, h, d) at base + t*stride_tok + h*stride_head + d, in
 * `in_dtype` (the reference takes fp32 after .float(); fp16 -> fp32 is exact,
 * so fp16 input gives the same bytes).  slot_mapping int32 [num_tokens]:
 * slot < 0 or slot >= num_blocks*block_size is skipped (the reference skips
 * negative slots).  signs fp32 [padded_dim] of +-1.  Bytes written per entry:
 * codes + norms; pad bytes are not touched.
 */
int tq_quantize_write_kv_cache(void* k_slab, void* v_slab,
                               const void* key, const void* value, int32_t in_dtype,
                               int64_t k_stride_tok, int64_t k_stride_head,
                               int64_t v_stride_tok, int64_t v_stride_head,
                               const float* signs, const int32_t* slot_mapping,
                               int64_t num_tokens, int32_t num_kv_heads,
                               int32_t head_dim, int32_t padded_dim,
                               int32_t block_size, int32_t ebs, int64_t num_blocks,
                               tq_stream_t stream);

/*
 * Split-KV GQA decode attention over the packed paged cache, one query token
 * per sequence: partials kernel + LSE merge with the inverse rotation.
 *
 * Replaces turboquant_v5::decode_v5_from_cache_paged_splitkv_ws
 * (reference csrc/src/decode_v5_tc_binding.cu:754-874: the v5 kernel
 * csrc/include/flashinfer_decode_turboquant_v5_tc.cuh:106-795 and
 * SplitKVCombineKernel csrc/include/flashinfer_decode_turboquant_combine.cuh:18-79),
 * called by TurboQuantFusedImpl.forward (turboquant/vllm_backend_fused.py:422-435).
 *
 * q: fp16, element (b, h, d) at q + b*q_stride_b + h*q_stride_h + d, d < pd;
 *    16-byte aligned, strides multiples of 8 elements, q_stride_h >= pd
 *    (head_dim < pd must be zero padded, as the reference backend does).
 * Sequence b's token t is page indices[indptr[b] + t/block_size], entry
 * t % block_size, for t < seq_lens[b]; block_size % 16 == 0.  Split s of
 * sequence b covers tokens [s*kv_chunk_size, min((s+1)*kv_chunk_size, seq_len)).
 * Pages outside [0, num_blocks) are treated as empty.
 * partition_o: fp32 [batch*num_splits, num_qo_heads, pd] and
 * partition_lse: fp32 [batch*num_splits, num_qo_heads] are workspace (the
 * partial rows are kept as fp16 in the first half of partition_o's bytes).
 * o: fp16 [batch, num_qo_heads, pd] contiguous, the attention output in the
 * original (unrotated) domain.  signs == NULL disables the rotation.
 * num_qo_heads / num_kv_heads must be an integer <= 16.
 */
int tq_decode_paged_splitkv(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                            const uint8_t* k_slab, const uint8_t* v_slab,
                            const int32_t* indices, const int32_t* indptr,
                            const int32_t* seq_lens, int32_t batch,
                            int32_t num_qo_heads, int32_t num_kv_heads,
                            int32_t head_dim, int32_t padded_dim,
                            int32_t block_size, int32_t ebs, int64_t num_blocks,
                            float sm_scale, const float* signs,
                            int32_t num_splits, int32_t kv_chunk_size,
                            float* partition_o, float* partition_lse, void* o,
                            tq_stream_t stream);

/*
 * tq_decode_paged_splitkv with the split plan made on the GPU (ragged
 * batches).  The reference sizes every sequence's splits from the batch's
 * max_len (turboquant/vllm_backend_fused.py:128-156), so at mixed lengths
 * most workgroups of short sequences sit idle; here each workgroup derives
 * the same plan from seq_lens: a unit size U (a multiple of 32 tokens, the
 * smallest with sum_b ceil(seq_len_b / U) no more than the grid's work
 * units) and its own (sequence, token range).  No host read, so a captured
 * graph stays valid while seq_lens change between replays.  Same inputs and
 * output as tq_decode_paged_splitkv, except:
 *   partition_o fp32 [max_rows, num_qo_heads, pd], partition_lse fp32
 *   [max_rows, num_qo_heads]: workspace; max_rows >= batch, and
 *   tq_decode_balanced_rows() gives the rows the plan uses at most;
 *   split_rows int32 [batch + 2] (written): sequence b's partial rows are
 *   split_rows[b] .. split_rows[b + 1] - 1, split_rows[batch + 1] = U.
 * batch <= 1024; sum of seq_lens < 2^30.
 */
int tq_decode_paged_balanced(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                             const uint8_t* k_slab, const uint8_t* v_slab,
                             const int32_t* indices, const int32_t* indptr,
                             const int32_t* seq_lens, int32_t batch,
                             int32_t num_qo_heads, int32_t num_kv_heads,
                             int32_t head_dim, int32_t padded_dim,
                             int32_t block_size, int32_t ebs, int64_t num_blocks,
                             float sm_scale, const float* signs, int32_t max_rows,
                             float* partition_o, float* partition_lse,
                             int32_t* split_rows, void* o, tq_stream_t stream);

/*
 * tq_decode_paged_balanced without workspace arguments and without any
 * allocation: the row table, partial LSEs and partial rows live in a
 * 16 MiB device array inside this library (one per GPU, kept until the
 * process ends), found once per device with hipGetSymbolAddress.  No
 * counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * The caller still passes inputs and o.  Limit: batch * num_qo_heads *
 * (padded_dim + 1) * 4 bytes of partials must fit the array (it is refused
 * with -22 otherwise; at most 1024 sequences); larger batches use fewer
 * rows per sequence, down to one.  Calls that overlap on one GPU (two
 * streams, or two threads) share the array and race: serialise them.
 */
int tq_decode_paged_balanced_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                     const uint8_t* k_slab, const uint8_t* v_slab,
                                     const int32_t* indices, const int32_t* indptr,
                                     const int32_t* seq_lens, int32_t batch,
                                     int32_t num_qo_heads, int32_t num_kv_heads,
                                     int32_t head_dim, int32_t padded_dim,
                                     int32_t block_size, int32_t ebs, int64_t num_blocks,
                                     float sm_scale, const float* signs, void* o,
                                     tq_stream_t stream);

/*
 * The first kernel of tq_decode_paged_balanced alone: the plan, the partial
 * rows (fp16 in partition_o) and partition_lse, and the row table in
 * split_rows; tq_combine_splits does not read a plan's rows, so this serves
 * timing and inspection of the partials kernel.
 */
int tq_decode_partials_balanced(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                const uint8_t* k_slab, const uint8_t* v_slab,
                                const int32_t* indices, const int32_t* indptr,
                                const int32_t* seq_lens, int32_t batch,
                                int32_t num_qo_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t padded_dim,
                                int32_t block_size, int32_t ebs, int64_t num_blocks,
                                float sm_scale, const float* signs, int32_t max_rows,
                                float* partition_o, float* partition_lse,
                                int32_t* split_rows, tq_stream_t stream);

/*
 * Partial rows tq_decode_paged_balanced uses at most for this geometry on
 * the current device (or -22).  Queries the device once per geometry.
 */
int tq_decode_balanced_rows(int32_t batch, int32_t num_qo_heads, int32_t num_kv_heads,
                            int32_t padded_dim);

/*
 * The first kernel of tq_decode_paged_splitkv alone (the reference's v5 split
 * kernel, v5_tc.cuh:106-795): writes the partial rows (normalised and,
 * when signs != NULL, rotated back to the original domain per split as
 * v5_tc.cuh:712-765 does; fp16 [batch*num_splits, num_qo_heads, pd] at the
 * start of partition_o) and partition_lse (natural log; -inf for an empty split) of
 * split s = tokens [s * kv_chunk_size, min((s + 1) * kv_chunk_size, seq_len)).
 */
int tq_decode_partials(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                       const uint8_t* k_slab, const uint8_t* v_slab,
                       const int32_t* indices, const int32_t* indptr,
                       const int32_t* seq_lens, int32_t batch,
                       int32_t num_qo_heads, int32_t num_kv_heads,
                       int32_t padded_dim, int32_t block_size, int32_t ebs,
                       int64_t num_blocks, float sm_scale, const float* signs,
                       int32_t num_splits, int32_t kv_chunk_size,
                       float* partition_o, float* partition_lse, tq_stream_t stream);

/*
 * The second kernel alone (reads the fp16 partial rows tq_decode_partials
 * leaves in partition_o, already in the original domain): LSE merge of the
 * splits of each sequence and the fp16 store into o.  Replaces
 * SplitKVCombineKernel (combine.cuh:18-79).  Splits with lse == -inf are
 * skipped; a sequence with no tokens gets zeros.  `signs` is not read (the
 * partials kernel applied the rotation); it stays in the signature for
 * callers of earlier versions.
 */
int tq_combine_splits(const float* partition_o, const float* partition_lse,
                      int32_t batch, int32_t num_splits, int32_t num_qo_heads,
                      int32_t padded_dim, const float* signs, void* o,
                      tq_stream_t stream);

/*
 * Read cached K/V back: the packed entries of tokens [0, num_tokens) of one
 * sequence (token t = page pages[t / block_size], entry t % block_size) as fp16
 * rows in the original domain, x = s * FWHT(c[code] * norm / sqrt(pd)) / sqrt(pd)
 * (no rotation when signs == NULL).  out_k / out_v: fp16, element (t, h, d) at
 * out + t * out_stride_tok + h * head_dim + d, d < head_dim.  Pages outside
 * [0, num_blocks) give zeros.
 *
 * Serves the prefill of a chunk whose sequence has cached context; the
 * reference's prefill (turboquant/vllm_backend_fused.py:335-371) attends the
 * fresh chunk only and has no counterpart.  The dequantization is the one its
 * decode reference applies (turboquant/triton_decode_ref.py:89-131).
 */
int tq_dequant_paged(const uint8_t* k_slab, const uint8_t* v_slab,
                     const int32_t* pages, int64_t num_tokens, int32_t num_kv_heads,
                     int32_t head_dim, int32_t padded_dim, int32_t block_size,
                     int32_t ebs, int64_t num_blocks, const float* signs,
                     void* out_k, void* out_v, int64_t out_stride_tok,
                     tq_stream_t stream);

/*
 * Causal GQA attention of a prefill chunk over fp16 K/V (head_dim 64, 128 or 256):
 * o[i, h] = softmax_j(q[i, h] . k[j, h / r] * sm_scale) v[j, h / r] over keys
 * j <= (kv_len - q_len) + i, r = num_qo_heads / num_kv_heads.  q, o: fp16
 * element (i, h, d) at base + i*stride_tok + h*stride_head + d; k, v: fp16
 * element (j, g, d) likewise.  Strides are multiples of 8 elements, bases
 * 16-byte aligned, 0 <= q_len <= kv_len.
 *
 * Replaces the flash-attn call of the reference's prefill
 * (flash_attn_varlen_func in TurboQuantFusedImpl.forward,
 * turboquant/vllm_backend_fused.py:335-371, which attends a chunk's fresh
 * K/V); the backend here calls it per request with the chunk's cached
 * context (tq_dequant_paged) in front of its fresh K/V.
 */
int tq_prefill_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                         const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                         const void* v, int64_t v_stride_tok, int64_t v_stride_head,
                         void* o, int64_t o_stride_tok, int64_t o_stride_head,
                         int32_t q_len, int32_t kv_len, int32_t num_qo_heads,
                         int32_t num_kv_heads, int32_t head_dim, float sm_scale,
                         tq_stream_t stream);

/*
 * tq_prefill_attention with a caller-owned workspace (no counterpart in the
 * reference, whose flash-attn call allocates its own): when the grid of
 * query blocks would leave CUs idle (a short chunk over a long context),
 * the keys of each query block are split over several workgroups, whose
 * results (fp16 O / row sum plus the reference max and row sum of every
 * row) go to `workspace` and are merged by a second kernel on the same
 * stream.  tq_prefill_workspace_bytes gives the size the current device's
 * plan needs (0: no split); with a null or smaller workspace the call runs
 * unsplit (same result).  The workspace must be 16-byte aligned; calls that
 * overlap on one workspace race.
 */
int tq_prefill_attention_ws(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                            const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                            const void* v, int64_t v_stride_tok, int64_t v_stride_head,
                            void* o, int64_t o_stride_tok, int64_t o_stride_head,
                            int32_t q_len, int32_t kv_len, int32_t num_qo_heads,
                            int32_t num_kv_heads, int32_t head_dim, float sm_scale,
                            void* workspace, int64_t workspace_bytes, tq_stream_t stream);
int64_t tq_prefill_workspace_bytes(int32_t q_len, int32_t kv_len, int32_t num_qo_heads,
                                   int32_t num_kv_heads, int32_t head_dim);

/*
 * The algorithm library's TurboQuantMSE quantizer (reference
 * turboquant/quantizer.py:63-118, TurboQuantMSE.quantize / .dequantize) on
 * the GPU, for fp32 vectors of dim <= padded_dim = next_pow2(dim) in
 * 64..1024 and bit_width 1..4.
 *
 * tq_mse_quantize: x fp32 [num_vectors, dim] (rows contiguous) ->
 *   norms fp32 [num_vectors] = max(||x||, 1e-8) and packed uint8
 *   [num_vectors, padded_dim / per] (per = 8 / bit_width, 2 for 3 bits;
 *   code i of a byte at bits i*bit_width), the codes being
 *   #{j : boundaries[j] < y_d} for y = FWHT(signs * pad(x / norm)) /
 *   sqrt(padded_dim).  boundaries: HOST fp32 array of 2^bit_width - 1
 *   values (the Codebook's, already scaled by 1/sqrt(padded_dim)).
 * tq_mse_dequantize: packed, norms -> out fp32 [num_vectors, dim] =
 *   (FWHT(centroids[code]) / sqrt(padded_dim) * signs)[:dim] * norm.
 *   centroids: HOST fp32 array of 2^bit_width values.
 * signs: device fp32 [padded_dim] of +-1.
 */
int tq_mse_quantize(const float* x, int64_t num_vectors, int32_t dim, int32_t padded_dim,
                    int32_t bit_width, const float* signs, const float* boundaries,
                    uint8_t* packed, float* norms, tq_stream_t stream);
int tq_mse_dequantize(const uint8_t* packed, const float* norms, int64_t num_vectors,
                      int32_t dim, int32_t padded_dim, int32_t bit_width, const float* signs,
                      const float* centroids, float* out, tq_stream_t stream);

/*
 * The algorithm library's TurboQuantProd (reference
 * turboquant/quantizer.py:121-158, with turboquant/qjl.py:28-63): the MSE
 * quantizer at mse_bit_width = bit_width - 1 (1..3 here), then QJL on the unit
 * residual.  The two d x d QJL products (sign(S r) and S^T z) are plain GEMMs
 * left to the caller's BLAS; these two calls are the rest of the algorithm.
 *
 * tq_prod_quantize: tq_mse_quantize's outputs, plus the MSE read-back
 *   x_hat = tq_mse_dequantize(packed, norms) (same fp32 bits), the residual
 *   norms fp32 [num_vectors] = max(||x - x_hat||, 1e-8) and residual_unit
 *   fp32 [num_vectors, dim] = (x - x_hat) / residual_norm (correctly rounded).
 *   centroids: HOST fp32 array of 2^mse_bit_width values.  residual_unit
 *   16-byte aligned.
 * tq_prod_dequantize: out fp32 [num_vectors, dim] = tq_mse_dequantize(packed,
 *   norms) + qjl_term * (fp32(sqrt(pi/2) / dim) * residual_norms), rounded in
 *   that order (the reference's torch expression), with qjl_term fp32
 *   [num_vectors, dim] = z S, z the +-1 QJL signs.
 */
int tq_prod_quantize(const float* x, int64_t num_vectors, int32_t dim, int32_t padded_dim,
                     int32_t mse_bit_width, const float* signs, const float* boundaries,
                     const float* centroids, uint8_t* packed, float* norms,
                     float* residual_unit, float* residual_norms, tq_stream_t stream);
int tq_prod_dequantize(const uint8_t* packed, const float* norms, const float* qjl_term,
                       const float* residual_norms, int64_t num_vectors, int32_t dim,
                       int32_t padded_dim, int32_t mse_bit_width, const float* signs,
                       const float* centroids, float* out, tq_stream_t stream);

/*
 * TurboQuantProd with the QJL projections on the GPU's matrix cores, for
 * padded_dim 64 or 128 (dim <= 128): the whole of quantizer.py:137-158 and
 * qjl.py:36-63 in one kernel each.  s_hi / s_lo (quantize) are the QJL
 * matrix S [dim, dim] as fp16 halves with S = hi + lo to 22 bits, zero-padded
 * to [padded_dim, padded_dim], row-major; st_hi / st_lo (dequantize) the same
 * of S^T.  16-byte aligned device arrays; qjl_signs 8-byte aligned (its
 * rows are read and written in 4- and 8-byte pieces when dim allows).
 *
 * tq_prod_quantize_qjl: tq_prod_quantize's packed, norms and residual_norms,
 *   and qjl_signs int8 [num_vectors, dim] = +1 where (S r)_j >= 0, else -1,
 *   r the unit residual (the reference's sign() with 0 -> +1).  The product
 *   is formed from the fp16 halves of S and r with fp32 accumulation, so a
 *   sign may differ from an fp32 GEMM's where |(S r)_j| is within about
 *   2^-22 |S_j| of 0.
 * tq_prod_dequantize_qjl: tq_prod_dequantize with qjl_term = z S formed
 *   in-kernel from qjl_signs (exact +-1 times the two halves of S).
 */
int tq_prod_quantize_qjl(const float* x, int64_t num_vectors, int32_t dim, int32_t padded_dim,
                         int32_t mse_bit_width, const float* signs, const float* boundaries,
                         const float* centroids, const void* s_hi, const void* s_lo,
                         uint8_t* packed, float* norms, int8_t* qjl_signs,
                         float* residual_norms, tq_stream_t stream);
int tq_prod_dequantize_qjl(const uint8_t* packed, const float* norms, const int8_t* qjl_signs,
                           const float* residual_norms, int64_t num_vectors, int32_t dim,
                           int32_t padded_dim, int32_t mse_bit_width, const float* signs,
                           const float* centroids, const void* st_hi, const void* st_lo,
                           float* out, tq_stream_t stream);

/*
 * Layer glue of the end-to-end harness, no counterpart in the
 * reference: in a vLLM deployment vLLM's own fused layer kernels do this.
 * fp16 tensors, rows contiguous, fp32 arithmetic inside.
 *
 * tq_e2e_add_rms_norm: x[r] += y[r] (fp16 add; skipped when y is NULL), then
 *   h[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * w (skipped when h is NULL);
 *   hidden a multiple of 8 up to 8192, 16-byte aligned rows.
 * tq_e2e_qk_norm_rope: for the q and k heads of each fused QKV row (q heads,
 *   then kv heads, then the v part, row stride qkv_row_stride elements):
 *   RMSNorm over the head's dims with q_w or k_w, rounded to fp16, then
 *   rotate-half RoPE with row positions[t] of the fp16 cos / signed-sin
 *   tables [table_rows, head_dim]: out[i] = n[i] cos[i] + n[(i + D/2) mod D]
 *   sin[i].  q_out [tokens, q_heads, D], k_out [tokens, kv_heads, D].  D
 *   even, <= 256.  A position outside [0, table_rows) gives NaN rows for its
 *   token (the positions live on the device; nothing is read past the tables).
 * tq_e2e_silu_mul: out[t, i] = silu(gate_up[t, i]) * gate_up[t, inter + i].
 */
int tq_e2e_add_rms_norm(void* x, const void* y, const void* w, void* h, int64_t rows,
                        int32_t hidden, float eps, tq_stream_t stream);
int tq_e2e_qk_norm_rope(const void* qkv, int64_t qkv_row_stride, const void* q_w,
                        const void* k_w, const void* cos_table, const void* sin_table,
                        int64_t table_rows, const int64_t* positions, int64_t tokens,
                        int32_t q_heads,
                        int32_t kv_heads, int32_t head_dim, float eps, void* q_out,
                        void* k_out, tq_stream_t stream);
int tq_e2e_silu_mul(const void* gate_up, void* out, int64_t rows, int32_t inter,
                    tq_stream_t stream);

/*
 * Diagnostic, no counterpart in the reference: with force_search != 0 the
 * quantize kernels (tq_mse_quantize, tq_prod_quantize*) take their codes by a
 * binary search over the boundaries instead of the one-lookup bin table they
 * use for symmetric codebooks, so that tests can check the two give the
 * same codes on the same inputs.  Process-wide; returns 0.
 */
int tq_diag_mse_bucketize(int32_t force_search);

/*
 * Diagnostic, no counterpart in the reference: tq_decode_partials at head
 * size 128 with 8 kv heads per workgroup (the configs[2] geometry) with parts
 * compiled out.  mode 1: the attention math (the same page walk, LDS copy
 * ring, waits, barriers and slot reads, plus the q setup, table build and
 * partial-row stores; zero partial rows).  mode 0: the bare copy ring (page
 * walk, copies, waits, barriers and slot reads; nothing stored).  Their
 * durations are the cost of the data movement alone (the bandwidth ceiling
 * of this kernel design).  Other geometries return -22.
 */
int tq_diag_decode_stream(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                          const uint8_t* k_slab, const uint8_t* v_slab,
                          const int32_t* indices, const int32_t* indptr,
                          const int32_t* seq_lens, int32_t batch,
                          int32_t num_qo_heads, int32_t num_kv_heads,
                          int32_t padded_dim, int32_t block_size, int32_t ebs,
                          int64_t num_blocks, float sm_scale, const float* signs,
                          int32_t num_splits, int32_t kv_chunk_size,
                          float* partition_o, float* partition_lse, int32_t mode,
                          tq_stream_t stream);

/*
 * Diagnostic, no counterpart in the reference: reads `bytes` (a multiple of
 * 16, 16-byte aligned) from device memory with non-temporal 16-byte loads,
 * a 2048 x 256 grid-strided stream; a lane stores to *sink only if the xor
 * of the words it read equals one constant.  Its duration is the HBM read rate a plain
 * stream reaches, beside which the decode kernel's copy ring is measured.
 */
int tq_diag_stream_read(const void* src, int64_t bytes, uint32_t* sink, tq_stream_t stream);

/* Message for the last non-zero return of a tq_* call on this thread. */
const char* tq_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int32_t tq_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TURBOQUANT_AMD_H */
