/*
 * libshardcompute_hip — C-ABI of the MI355X (gfx950) kernels behind ShardCompute's
 * per-rank quantized inference hot path.
 *
 * Conventions for every entry point:
 *  - Pointers are device pointers (hipMalloc / torch-ROCm tensors), row-major and
 *    contiguous.  bf16 values are passed as uint16_t bit patterns.
 *  - Quantized weights use MLX's affine format: uint32 words holding 32/bits codes
 *    of consecutive columns, least significant first; one bf16 scale and bias per
 *    group of `group_size` columns; dequantized value = scale * q + bias.
 *  - Work is enqueued on `hip_stream` (NULL = the null stream) and never
 *    synchronised; outputs are valid once that stream reaches the work.
 *  - Return 0 on success, a negative status otherwise (-1 bad argument,
 *    -2 unsupported configuration, -3 HIP runtime error); sc_last_error() then
 *    holds a message (thread-local, valid until the next failing call).
 *  - The kernels allocate nothing per call.  The split-K path of sc_qmm_bf16 (and of
 *    the products inside sc_qmm_rmsnorm_bf16 / sc_qmm_swiglu_bf16 / sc_qmm_add_rmsnorm_bf16:
 *    9-160 rows, and larger products whose 256-wide tiles fill at most half the GPU) uses a
 *    library-owned scratch per device, allocated on first need and grown (with a
 *    device synchronisation) when a larger shape arrives: calls that overlap on one
 *    device (concurrent streams) race on it, and the first call of a new largest
 *    shape must not happen under stream capture.  sc_qmm_bf16_noalloc is the
 *    variant that never allocates.
 */
#ifndef SHARDCOMPUTE_HIP_H
#define SHARDCOMPUTE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SC_ABI_VERSION 13

/* Kernel selection for sc_qmm_bf16_path. */
#define SC_QMM_PATH_AUTO 0 /* M <= 16: GEMV or band kernel (8-16 rows, by shape);
                              17-160: band kernel; above: GEMM                  */
#define SC_QMM_PATH_GEMV 1 /* fused dequant-GEMV (decode batches, M <= 32)      */
#define SC_QMM_PATH_GEMM 2 /* LDS-staged dequant -> bf16 MFMA GEMM (prefill)     */
#define SC_QMM_PATH_BAND 3 /* weight-streaming band kernel (M <= 256)            */

/* ABI version of the loaded library (SC_ABI_VERSION at build time). */
int sc_abi_version(void);

/* Message of the last failing call on this thread. */
const char *sc_last_error(void);

/*
 * y[M, N] = bf16( x[M, K] @ dequant(wq, scales, biases)^T ), then, when
 * bias_or_null is given, y = bf16(y + bias[N]).  fp32 accumulation.
 *   x      bf16 [M, K], 16-byte aligned      wq  uint32 [N, K*bits/32], 16-byte aligned
 *   scales bf16 [N, K/group_size]            biases bf16 [N, K/group_size]
 *   bits in {4, 8}, group_size == 64, K % group_size == 0.
 * Replaces mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size, bits)
 * plus the "+ self.bias" that follows it:
 *   src/shardcompute/parallel/quantized_linear.py:168-180   (QuantizedColumnParallelLinear.forward)
 *   src/shardcompute/parallel/quantized_linear.py:206-217   (.forward_sync)
 *   src/shardcompute/parallel/quantized_linear.py:435-443   (QuantizedRowParallelLinear.forward)
 *   src/shardcompute/parallel/quantized_linear.py:472-480   (.forward_partial)
 *   src/shardcompute/parallel/transformer.py:639-647, 971-979 (pipeline LinearLayer / lm_head)
 *   src/shardcompute/model/quantization.py:67-75            (QuantizedWeight.matmul)
 */
int sc_qmm_bf16(const uint16_t *x, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                const uint16_t *bias_or_null, uint16_t *y, int64_t M, int64_t N, int64_t K, int bits,
                int group_size, void *hip_stream);

/*
 * sc_qmm_bf16 with an explicit kernel choice (SC_QMM_PATH_*): lets tests and
 * benchmarks run both kernels on the same shape.  Same reference call sites.
 */
int sc_qmm_bf16_path(const uint16_t *x, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                     const uint16_t *bias_or_null, uint16_t *y, int64_t M, int64_t N, int64_t K, int bits,
                     int group_size, int path, void *hip_stream);

/*
 * sc_qmm_bf16 on the band kernel (M <= 256, K a multiple of 512) with its plan
 * pinned: waves per workgroup (4 or 8; 0 = automatic) and K splits (0 = automatic).
 * For measurements of the plan; results do not depend on it beyond the split-K
 * summation order.  Same reference call sites as sc_qmm_bf16.
 */
int sc_qmm_bf16_band(const uint16_t *x, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                     const uint16_t *bias_or_null, uint16_t *y, int64_t M, int64_t N, int64_t K, int bits,
                     int group_size, int waves, int ksplit, void *hip_stream);

/* Size of the device array that sc_qmm_bf16_noalloc's split-K partials live in. */
#define SC_QMM_NOALLOC_SCRATCH_BYTES (4u << 20)

/*
 * sc_qmm_bf16 that never allocates device memory, for callers that cannot call
 * hipMalloc: code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation.  No counterpart in the reference (mx.quantized_matmul
 * allocates its output; this entry point allocates nothing at all).  Same
 * arguments, kernels and results as sc_qmm_bf16, bit for bit.  Where the 9-160-row
 * band kernel or the 9-32-row GEMV splits K across workgroups, its fp32 partials go
 * to a file-scope device array of SC_QMM_NOALLOC_SCRATCH_BYTES (one per GPU, held
 * until the process ends) instead of the library's growable buffer.  A shape whose
 * partials (splits * M * N floats) exceed it runs on the next kernel that needs no
 * scratch (the 32-column GEMV or the GEMM): within the same 1e-2 of the exact product
 * but not bit for bit equal to sc_qmm_bf16.  The array's
 * address is looked up on the first call on each device (no allocation, no
 * synchronisation).  Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (concurrent streams) race.  Each launch writes every
 * partial it reads, so nothing needs clearing between calls.
 */
int sc_qmm_bf16_noalloc(const uint16_t *x, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                        const uint16_t *bias_or_null, uint16_t *y, int64_t M, int64_t N, int64_t K, int bits,
                        int group_size, void *hip_stream);

/*
 * Vocab-sharded bf16 row gather: for t < T,
 *   out[t, :] = table[ids[t] - vocab_start, :]  if vocab_start <= ids[t] < vocab_start + v_local
 *             = +0.0                            otherwise,
 * bit for bit.  ids are int32 (ids_is_int64 = 0) or int64; table bf16 [v_local, D].
 * Implements the mask/clip/take/where of
 *   src/shardcompute/parallel/embedding.py:322-356 (QuantizedParallelEmbedding.forward)
 * on the bf16 table of VocabParallelEmbedding (a stub at embedding.py:397-418), and the
 * plain lookup mx.take(weight, ids, axis=0) of ParallelEmbedding (embedding.py:131-132,
 * 164-165) when vocab_start = 0 and v_local = vocab_size.
 */
int sc_vocab_gather_bf16(const void *ids, int ids_is_int64, int64_t T, const uint16_t *table, int64_t v_local,
                         int64_t D, int64_t vocab_start, uint16_t *out, void *hip_stream);

/*
 * Vocab-sharded gather of a quantized table, dequantized to bf16:
 *   out[t, k] = bf16(scales[r, k/gs] * q[r, k] + biases[r, k/gs]),  r = ids[t] - vocab_start,
 * for in-shard ids, +0.0 rows otherwise.  wq uint32 [v_local, D*bits/32], D % 64 == 0,
 * out 16-byte aligned.  Replaces the take + mx.dequantize + where of
 *   src/shardcompute/parallel/embedding.py:322-356.
 */
int sc_qembed_gather_bf16(const void *ids, int ids_is_int64, int64_t T, const uint32_t *wq,
                          const uint16_t *scales, const uint16_t *biases, int64_t v_local, int64_t D,
                          int64_t vocab_start, int bits, int group_size, uint16_t *out, void *hip_stream);

/*
 * out[rows, K] = bf16(scales * q + biases) for a whole quantized matrix.  Replaces
 * mx.dequantize at src/shardcompute/parallel/embedding.py:369-379 and
 * src/shardcompute/model/quantization.py:44-52.
 */
int sc_dequantize_bf16(const uint32_t *wq, const uint16_t *scales, const uint16_t *biases, int64_t rows,
                       int64_t K, int bits, int group_size, uint16_t *out, void *hip_stream);

/*
 * MLX affine quantizer on the GPU: fp32 w [rows, K] -> wq uint32 [rows, K*bits/32],
 * bf16 scales/biases [rows, K/64] (edge-preserving rule, fp32 arithmetic, RNE).
 * Replaces mx.quantize at src/shardcompute/parallel/quantized_linear.py:116-120, 353-357
 * and src/shardcompute/parallel/embedding.py:303-307 (followed by a bf16 cast of the
 * scales and biases).
 */
int sc_quantize_affine(const float *w, int64_t rows, int64_t K, int bits, int group_size, uint32_t *wq,
                       uint16_t *scales, uint16_t *biases, void *hip_stream);

/*
 * The projection that feeds a residual add and the next RMSNorm:
 *   y = qmm(x) (+ bias after rounding), h = bf16(y + residual), xn = RMSNorm(h) * w.
 * h_out [M, N] receives h and xn_out [M, N] xn (N a multiple of 8 up to 16384;
 * residual, norm_weight, h_out, xn_out and the bias 16-byte aligned; h_out and xn_out
 * overlap neither each other nor the inputs).  Where the product splits K (the
 * 9-160-row kernels) the norm's pass sums the partials itself, one launch in place
 * of the split-K pass and the norm; otherwise the product writes y into xn_out and
 * the pass reads it there.  Bit for bit sc_qmm_bf16 followed by sc_rms_norm_bf16
 * with that residual.  Replaces o_proj / down_proj with the residual add and the
 * next layernorm when the all-reduce between them is the identity
 * (src/shardcompute/parallel/transformer.py:246 then 250, and 252 then the next
 * layer's 239; quantized_linear.py:435-443 at world_size 1).
 */
int sc_qmm_add_rmsnorm_bf16(const uint16_t *x, const uint32_t *wq, const uint16_t *scales, const uint16_t *biases,
                            const uint16_t *bias_or_null, const uint16_t *residual, const uint16_t *norm_weight,
                            float eps, uint16_t *h_out, uint16_t *xn_out, int64_t M, int64_t N, int64_t K, int bits,
                            int group_size, void *hip_stream);

/*
 * y = qmm(xn) with xn = RMSNorm(x + residual) (residual optional): the
 * normalisation that precedes a projection, applied by the decode GEMV while it
 * stages its input rows (M <= 8), else by the standalone sc_rms_norm_bf16 first.
 * On return xn_out [M, K] holds xn and, when a residual is given and h_out_or_null
 * is not null, h_out [M, K] holds x + residual.  Outputs must not overlap x or the
 * residual.  Replaces RMSNorm.__call__ (src/shardcompute/parallel/transformer.py:46-61)
 * followed by the first projection that reads it (attention.py:406-408 after
 * transformer.py:240, mlp.py:241-242 after transformer.py:249, and the lm_head
 * after transformer.py:562).
 */
int sc_qmm_rmsnorm_bf16(const uint16_t *x, const uint16_t *residual_or_null, const uint16_t *norm_weight, float eps,
                        uint16_t *h_out_or_null, uint16_t *xn_out, const uint32_t *wq, const uint16_t *scales,
                        const uint16_t *biases, const uint16_t *bias_or_null, uint16_t *y, int64_t M, int64_t N,
                        int64_t K, int bits, int group_size, void *hip_stream);

/* Bytes of the sc_decode_head_bf16 workspace. */
#define SC_DECODE_HEAD_WORKSPACE_BYTES 16

/*
 * The greedy tail of a decode step: logits = qmm(RMSNorm(x + residual)) exactly
 * as sc_qmm_rmsnorm_bf16 (same arguments, logits [M, N] in place of y), then
 * ids / tokens exactly as sc_argmax_bf16 on the logits, then counters[i] += 1 for
 * i < n_counters as sc_add_i32 (step_or_null may point into the counters: the
 * token column is read before they advance).  At M = 1 the decode GEMV selects the
 * token while it writes the logits (its workgroups max their outputs' keys into
 * the workspace; the last to finish writes the token and advances the counters),
 * so no second pass over the logits runs; otherwise the three steps run in turn.
 * workspace: SC_DECODE_HEAD_WORKSPACE_BYTES, 16-byte aligned, zero before the
 * first call; every call leaves it zero.  Calls that share a workspace must not
 * overlap (one stream).  Replaces the final norm and lm_head of the decode step
 * (src/shardcompute/parallel/transformer.py:562, :575) with the greedy mx.argmax of
 * src/shardcompute/worker/executor.py:276-278 and the cache-length bookkeeping of
 * executor.py:134-136.
 */
int sc_decode_head_bf16(const uint16_t *x, const uint16_t *residual_or_null, const uint16_t *norm_weight, float eps,
                        uint16_t *h_out_or_null, uint16_t *xn_out, const uint32_t *wq, const uint16_t *scales,
                        const uint16_t *biases, const uint16_t *bias_or_null, uint16_t *logits, int64_t M, int64_t N,
                        int64_t K, int bits, int group_size, int32_t *ids, int32_t *tokens_or_null,
                        int64_t tokens_stride, int64_t tokens_cols, const int32_t *step_or_null,
                        int32_t *counters_or_null, int64_t n_counters, void *workspace, int64_t workspace_bytes,
                        void *hip_stream);

/*
 * act = silu(gate) * up for the stacked gate|up weight wq [2I, K*bits/32] (gate rows
 * first; scales/biases [2I, K/64], bias_or_null [2I]) applied to x, or to
 * xn = RMSNorm(x + residual) when norm_weight_or_null is given (xn_out and, with a
 * residual, h_out receive xn and x + residual as for sc_qmm_rmsnorm_bf16).  The
 * decode GEMV (M <= 8) pairs gate row i with up row I + i inside one tile and writes
 * act [M, I] directly; at 9-160 rows (band kernel, K a multiple of 512, chosen by
 * shape up to 32 rows; else the split-K GEMV) the split-K pass rounds gate and up to bf16 (bias after
 * rounding) and writes act [M, I]; above that the GEMM pairs gate and up columns in its tiles
 * and writes act itself (I a multiple of 16).  gate_up_scratch [M, 2I] is required but
 * used only where none of these applies: then the product goes there and the
 * standalone sc_silu_mul_bf16 follows (the same values).  Outputs must not overlap
 * the inputs.
 * Replaces ParallelMLP.forward's gate/up projections and activation
 * (src/shardcompute/parallel/mlp.py:241-245), after the post-attention layernorm
 * (transformer.py:249-250).
 */
int sc_qmm_swiglu_bf16(const uint16_t *x, const uint16_t *residual_or_null, const uint16_t *norm_weight_or_null,
                       float eps, uint16_t *h_out_or_null, uint16_t *xn_out_or_null, const uint32_t *wq,
                       const uint16_t *scales, const uint16_t *biases, const uint16_t *bias_or_null, uint16_t *act_out,
                       uint16_t *gate_up_scratch, int64_t M, int64_t I, int64_t K, int bits, int group_size,
                       void *hip_stream);

/* ------------------------------------------------------------------------------
 * Decoder wiring around the quantized linears.  The cache length (the number of
 * positions already in the KV cache) is read from device memory, so a decode step
 * captured once in a HIP graph replays at every position.
 *
 * KV cache per layer, capacity T_cap (a multiple of 32), zero-initialised:
 *   k_cache   [B, Hkv, T_cap, D] bf16
 *   v_cache_t [B, Hkv, D, T_cap] bf16 (values transposed)
 * ---------------------------------------------------------------------------- */

/*
 * h = x + residual (bf16, when residual_or_null is given; written to h_out_or_null
 * when that is given) and y = (h / sqrt(mean(h*h) + eps)) * weight, row-wise over
 * D (a multiple of 8, at most 16384).  Replaces RMSNorm.__call__ at
 * src/shardcompute/parallel/transformer.py:46-61 and the residual adds of
 * ParallelTransformerBlock.forward at transformer.py:246 and :252.
 */
int sc_rms_norm_bf16(const uint16_t *x, const uint16_t *residual_or_null, const uint16_t *weight, uint16_t *y,
                     uint16_t *h_out_or_null, int64_t rows, int64_t D, float eps, void *hip_stream);

/*
 * RoPE on the q and k heads of the fused projection rows qkv [B*S, qkv_stride]
 * (q heads, then k heads, then v heads, each D wide).  Token s of each sequence
 * goes to cache slot cache_len[0] + s and is rotated for position
 * cache_len[0] + s + pos_offset (rotate-half, fp32 tables cos_t/sin_t
 * [table_len, D/2]); rotated q is written back in place, rotated k and v are
 * appended to the cache.  Replaces RoPE.__call__ / RoPE._rotate and the KV
 * concatenation of ParallelAttention.forward at
 * src/shardcompute/parallel/attention.py:94-151 and :421-435.
 */
int sc_rope_append_kv_bf16(uint16_t *qkv, int64_t qkv_stride, int64_t B, int64_t S, int64_t H, int64_t Hkv,
                           int64_t D, const float *cos_t, const float *sin_t, int64_t table_len, uint16_t *k_cache,
                           uint16_t *v_cache_t, int64_t T_cap, const int32_t *cache_len, int64_t pos_offset,
                           void *hip_stream);

/* Bytes of workspace sc_attention_bf16 needs for these sizes (0: none). */
int64_t sc_attention_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t Hkv, int64_t D, int64_t T_cap);

/*
 * Causal GQA attention of S new positions per sequence against the cache, which
 * holds cache_len[0] earlier positions followed by the S new ones (appended by
 * sc_rope_append_kv_bf16 with the same cache_len): out = softmax(q k^T * scale +
 * causal mask) v, q head h reading KV head h / (H / Hkv).  q rows at
 * q + (b*S + s)*q_stride + h*D, output rows likewise with out_stride.  D is 64 or
 * 128.  Replaces the score / mask / softmax / value steps of
 * ParallelAttention.forward at src/shardcompute/parallel/attention.py:437-466.
 */
int sc_attention_bf16(const uint16_t *q, int64_t q_stride, const uint16_t *k_cache, const uint16_t *v_cache_t,
                      int64_t T_cap, const int32_t *cache_len, uint16_t *out, int64_t out_stride, int64_t B,
                      int64_t S, int64_t H, int64_t Hkv, int64_t D, float scale, void *workspace,
                      int64_t workspace_bytes, void *hip_stream);

/*
 * sc_attention_bf16 with an additive mask: scores q k^T * scale + mask[b, h, s, t]
 * + causal mask, softmax, times v.  Mask element (b, h, s, t) (q head h, new
 * position s, key t of the cache_len[0] + S keys) is the fp32 at mask + b*mask_stride_b
 * + h*mask_stride_h + s*mask_stride_s + t*mask_stride_t; strides are in elements and
 * non-negative, 0 broadcasting a dimension, and the caller sizes the mask for every
 * key t a position sees.  A row whose visible scores are all -inf gives NaN, as the
 * reference's softmax does.  Workspace as for sc_attention_bf16.  Replaces
 * attention.py:449-450 (attn_scores + attention_mask) together with the steps
 * sc_attention_bf16 replaces (src/shardcompute/parallel/attention.py:437-466).
 */
int sc_attention_masked_bf16(const uint16_t *q, int64_t q_stride, const uint16_t *k_cache, const uint16_t *v_cache_t,
                             int64_t T_cap, const int32_t *cache_len, uint16_t *out, int64_t out_stride, int64_t B,
                             int64_t S, int64_t H, int64_t Hkv, int64_t D, float scale, const float *mask,
                             int64_t mask_stride_b, int64_t mask_stride_h, int64_t mask_stride_s,
                             int64_t mask_stride_t, void *workspace, int64_t workspace_bytes, void *hip_stream);

/* Bytes of workspace sc_attention_decode_bf16 needs (0: none). */
int64_t sc_attention_decode_workspace_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t D, int64_t T_cap);

/*
 * One decode step of attention (one new position per sequence): RoPE of the q and
 * k heads of qkv row b (rotary position cache_len[0] + pos_offset, tables as for
 * sc_rope_append_kv_bf16), append of the rotated k and of v at cache slot
 * cache_len[0], and causal GQA attention of the new position over the cache
 * (cache_len[0] + 1 keys); out row b at out + b*out_stride.  Equal to
 * sc_rope_append_kv_bf16 followed by sc_attention_bf16 with S = 1 (same cache
 * contents afterwards; the output within float rounding, the new key entering the
 * softmax from registers), with one launch fewer.  H / Hkv <= 16, D 64 or 128.
 * The qkv row is not modified.  Replaces ParallelAttention.forward's RoPE, KV
 * concatenation and attention for one token
 * (src/shardcompute/parallel/attention.py:421-466).
 */
int sc_attention_decode_bf16(const uint16_t *qkv, int64_t qkv_stride, int64_t B, int64_t H, int64_t Hkv, int64_t D,
                             const float *cos_t, const float *sin_t, int64_t table_len, uint16_t *k_cache,
                             uint16_t *v_cache_t, int64_t T_cap, const int32_t *cache_len, int64_t pos_offset,
                             float scale, uint16_t *out, int64_t out_stride, void *workspace,
                             int64_t workspace_bytes, void *hip_stream);

/*
 * sc_attention_decode_bf16 with an additive mask: every score of row b's new
 * position, q head h and key t (the cache_len[0] + 1 keys, the new one included)
 * gets mask[b, h, t] added after the scaling, as sc_attention_masked_bf16 adds it
 * (element at mask + b*mask_stride_b + h*mask_stride_h + t*mask_stride_t, fp32,
 * strides non-negative, 0 broadcasting).  Same cache contents as
 * sc_rope_append_kv_bf16; the output equals sc_attention_masked_bf16 with S = 1
 * within float rounding, in one launch (plus the range merge) instead of two.  A row
 * whose visible scores are all -inf gives NaN.  Replaces ParallelAttention.forward's
 * RoPE, KV concatenation, attention and attention_mask addition for one token
 * (src/shardcompute/parallel/attention.py:421-466, 449-450).
 */
int sc_attention_decode_masked_bf16(const uint16_t *qkv, int64_t qkv_stride, int64_t B, int64_t H, int64_t Hkv,
                                    int64_t D, const float *cos_t, const float *sin_t, int64_t table_len,
                                    uint16_t *k_cache, uint16_t *v_cache_t, int64_t T_cap, const int32_t *cache_len,
                                    int64_t pos_offset, float scale, const float *mask, int64_t mask_stride_b,
                                    int64_t mask_stride_h, int64_t mask_stride_t, uint16_t *out, int64_t out_stride,
                                    void *workspace, int64_t workspace_bytes, void *hip_stream);

/*
 * out[rows, I] = silu(gate) * up for gate_up [rows, 2I] (gate columns first), with
 * silu(g) = g / (1 + exp(-g)).  Replaces the activation step of ParallelMLP.forward
 * at src/shardcompute/parallel/mlp.py:161-162 and :241-245.
 */
int sc_silu_mul_bf16(const uint16_t *gate_up, int64_t rows, int64_t I, uint16_t *out, void *hip_stream);

/* Activation kinds of sc_act_bf16 (ParallelMLP's activation names). */
#define SC_ACT_SILU 0       /* "silu" / "swish": x / (1 + exp(-x))                        */
#define SC_ACT_GELU 1       /* "gelu": x * sigmoid(1.702 x)                               */
#define SC_ACT_GELU_NEW 2   /* "gelu_new": 0.5 x (1 + tanh(0.79788456 (x + 0.044715 x^3))) */
#define SC_ACT_RELU 3       /* "relu": max(x, 0)                                          */
#define SC_ACT_GELU_EXACT 4 /* "gelu_exact": 0.5 x (1 + erf(x / sqrt(2)))                 */

/*
 * The MLP activation of any kind: gated, out[rows, I] = f(gate) * up for
 * in = gate|up [rows, 2I] (gate columns first); ungated, out[rows, I] = f(in[rows, I])
 * (out may equal in).  fp32 arithmetic, one bf16 rounding.  I a multiple of 8,
 * 16-byte aligned pointers.  Replaces the activation step of ParallelMLP.forward,
 * gated and ungated, for every activation it accepts:
 *   src/shardcompute/parallel/mlp.py:159-180 (the activations), :236-250 (their use).
 */
int sc_act_bf16(const uint16_t *in, int64_t rows, int64_t I, int kind, int gated, uint16_t *out, void *hip_stream);

/*
 * out[r, d] = bf16(x[r, d] + bias[d]) for x [rows, D] (out may equal x): the
 * LayerNorm-style bias of RMSNorm.__call__, src/shardcompute/parallel/transformer.py:
 * 57-59, added to the normalised, scaled row.  D a multiple of 8, 16-byte aligned.
 */
int sc_add_row_bias_bf16(const uint16_t *x, int64_t rows, int64_t D, const uint16_t *bias, uint16_t *out,
                         void *hip_stream);

/*
 * ids[r] = first index of the maximum of logits row r (NaN counts as the maximum,
 * -0.0 equals +0.0).  When tokens_or_null is given the id is also stored at
 * tokens[r*tokens_stride + c] with c = (step_or_null ? step[0] : 0), provided
 * 0 <= c < tokens_cols (otherwise only ids is written).  Replaces the greedy
 * mx.argmax of ParallelExecutor.generate at src/shardcompute/worker/executor.py:276-278.
 */
int sc_argmax_bf16(const uint16_t *logits, int64_t rows, int64_t V, int32_t *ids, int32_t *tokens_or_null,
                   int64_t tokens_stride, int64_t tokens_cols, const int32_t *step_or_null, void *hip_stream);

/*
 * out = a + b elementwise in bf16 (n a multiple of 8): the residual adds of
 * ParallelTransformerBlock.forward at src/shardcompute/parallel/transformer.py:246, :252
 * where no normalisation follows.
 */
int sc_add_bf16(const uint16_t *a, const uint16_t *b, uint16_t *out, int64_t n, void *hip_stream);

/*
 * counters[i] += delta for i < n (n <= 64), on the stream: advances the device-side
 * cache length / step counters between graph replays.  Stands in for the
 * cache-length bookkeeping of src/shardcompute/worker/executor.py:134-136 (the cache
 * grows by the step's sequence length).
 */
int sc_add_i32(int32_t *counters, int64_t n, int32_t delta, void *hip_stream);

/*
 * One batch-1 decode step of the whole decoder trunk in one persistent launch.
 *
 * Replaces the per-token pass through the layer stack at one position,
 * src/shardcompute/parallel/transformer.py:537-559 (embed_tokens, then per layer
 * ParallelTransformerBlock.forward :214-254 = RMSNorm, ParallelAttention.forward
 * attention.py:381-471 with QuantizedColumnParallelLinear q/k/v and
 * QuantizedRowParallelLinear o_proj, RMSNorm, ParallelMLP.forward mlp.py:228-254),
 * at world_size 1 or one rank's shard with the all-reduces as identity, every
 * projection an MLX-affine g64 quantized matmul without linear bias.
 *
 * Per layer the caller passes the q|k|v rows stacked into one matrix
 * [(H + 2 Hkv) * D, hidden], o [hidden, H * D], gate|up stacked [2 I, hidden] (gate
 * rows first), down [hidden, I], the two norm weights and the layer's cache
 * (batch 1: keys [Hkv, T_cap, D], values transposed [Hkv, D, T_cap]).
 * `counters[0]` is the new token's cache slot (read on the device at launch),
 * `ids[0]` its token id.  After the launch `h_out` holds the residual stream that
 * the final RMSNorm + lm_head read, and every layer's cache holds the new position.
 *
 * sc_decode_plan_create validates the shapes (head_dim 128 with at most 4 query heads
 * per kv head, or head_dim 64 with at most 8; widths multiples of 512 up to 16384,
 * group size 64, the attention rows and
 * key ranges splitting over the device's CUs, the whole working set within one CU's
 * LDS), uploads the per-layer pointer table and allocates the plan's exchange buffers
 * (a few MB; -2 for a shape it does not take); sc_decode_plan_run enqueues the
 * launch on `hip_stream` (capturable: it allocates nothing and calls no memset).
 * Launches of one plan must not overlap.  sc_decode_plan_status copies the plan's
 * status word (0: every launch completed; nonzero: a launch gave up after a bounded
 * wait, outputs invalid) to the host, synchronously.
 */
typedef struct sc_decode_layer {
    const uint32_t *wq_qkv; const uint16_t *s_qkv, *b_qkv;
    const uint32_t *wq_o; const uint16_t *s_o, *b_o;
    const uint32_t *wq_gu; const uint16_t *s_gu, *b_gu;
    const uint32_t *wq_down; const uint16_t *s_down, *b_down;
    const uint16_t *ln_in, *ln_post;
    uint16_t *kc, *vt;
} sc_decode_layer;

typedef struct sc_decode_model {
    int num_layers, hidden, intermediate, num_heads, num_kv_heads, head_dim, bits, group_size;
    float eps, scale;                 /* RMSNorm epsilon; attention scale (1/sqrt(head_dim)) */
    const uint16_t *embed;            /* bf16 [vocab_local, hidden] */
    int64_t vocab_start, vocab_local;
    const float *cos_t, *sin_t;       /* fp32 [table_len, head_dim / 2] */
    int table_len, pos_offset;
    int T_cap;                        /* cache capacity (multiple of 32) */
    const int32_t *counters;
    const int32_t *ids;
    uint16_t *h_out;                  /* bf16 [hidden] */
} sc_decode_model;

int sc_decode_plan_create(const sc_decode_model *model, const sc_decode_layer *layers, void **plan_out);
int sc_decode_plan_run(void *plan, void *hip_stream);
int sc_decode_plan_status(void *plan, uint32_t *status);
void sc_decode_plan_destroy(void *plan);

/*
 * Per-op timeline of the whole-trunk launch: the fused counterpart of the per-layer
 * timing of ParallelExecutor.forward_with_timing (src/shardcompute/worker/executor.py:
 * 155-227), which cannot bracket layers inside one launch with host clocks.
 * sc_decode_plan_trace(plan, 1) allocates a stamp buffer (not under stream capture)
 * and makes later launches record, per workgroup w and op j (op 0 the embedding,
 * then 6 per layer: q|k|v, attention, key-range merge, o, gate|up, down), the
 * 100 MHz real-time clock at four points: the op's items all computed (k = 0), its
 * output published (1), its input polled (2) and staged (3), at
 * stamps[(w * ops + j) * 4 + k]; (plan, 0) stops recording for later launches.  The
 * buffer stays allocated until sc_decode_plan_destroy, so a graph captured while
 * tracing was on may still be replayed.  sc_decode_plan_read_trace copies the stamps
 * of the last launch that recorded (n entries at least workgroups * ops * 4; stamps
 * may be null to query the sizes), synchronously.
 */
int sc_decode_plan_trace(void *plan, int enable);
int sc_decode_plan_read_trace(void *plan, uint32_t *stamps, int64_t n, int *workgroups, int *ops);

#ifdef __cplusplus
}
#endif

#endif /* SHARDCOMPUTE_HIP_H */
