/*
 * nqamd_shell.h — C ABI of the decoder-shell kernels that run around the
 * packed linears in batch-1 autoregressive decode (Qwen3 geometry: RMSNorm,
 * per-head q/k RMSNorm, rotate-half RoPE, grouped-query attention over a KV
 * cache, SiLU-gated MLP, untied bf16 output projection, greedy selection).
 *
 * Conventions are those of nqamd.h: device pointers owned by the caller,
 * `stream` is a hipStream_t passed as void*, nothing allocates, frees or
 * synchronises, the return value is an nq_status.
 *
 * Positions live in device memory (`position`, one int32 = the cache row of
 * the first token of the call) so that a captured decode step can be replayed
 * without rebuilding its kernel arguments; nq_greedy_select advances it.
 *
 * KV cache layout, per layer: [kv_heads][max_positions][head_dim] in
 * cache_dtype (F16/BF16/F32). RoPE tables: [max_positions][head_dim / 2] fp32,
 * cos and sin of position * inv_freq[i].
 */
#ifndef NQAMD_SHELL_H
#define NQAMD_SHELL_H

#include <stddef.h>
#include <stdint.h>

#include "nqamd.h"

#ifdef __cplusplus
extern "C" {
#endif

/* out[t, :] = table[ids[t], :] (* scale[0] when scale is not NULL) as fp32.
 * table dtype F32/F16/BF16, hidden % 8 == 0. An id outside [0, vocab) gives a
 * row of NaN (no out-of-range read). Replaces launch_bfloat16_embedding
 * (src/nanoquant/runtime/cuda_kernels.py:620-681). */
int nq_embedding(const int64_t* ids, int64_t tokens, const void* table, int32_t table_dtype,
                 int64_t vocab, int64_t hidden, const float* scale, float* out, void* stream);

/* nq_embedding that also writes, for each output row, the sums of squares of
 * its 16-column groups: slots [tokens][hidden / 16] fp32, hidden % 16 == 0.
 * These are the row statistics the NQ_INPUT_RMSNORM input of
 * nq_linear_batch_fused reads (norm_slots), so the first layer's projections
 * take the embedding's output with the RMSNorm folded in, as later layers take
 * the residual. No reference counterpart: the reference's embedding
 * (src/nanoquant/runtime/cuda_kernels.py:620-681) is followed by a separate
 * RMSNorm. */
int nq_embedding_slots(const int64_t* ids, int64_t tokens, const void* table, int32_t table_dtype,
                       int64_t vocab, int64_t hidden, const float* scale, float* out, float* slots,
                       void* stream);

/* Residual add and RMSNorm, one row per token:
 *   residual[t, :] += delta[t, :]                      (skipped when delta is NULL)
 *   out[t, :] = weight * (residual[t, :] * rsqrt(mean(residual[t, :]^2) + eps))
 * residual fp32 (updated in place), delta F32/F16/BF16, weight F32/F16/BF16,
 * out F32/F16/BF16, hidden % 8 == 0 and hidden <= 16384. Replaces the residual adds of
 * Qwen3DecoderLayer.forward and Qwen3RMSNorm (the reference runs the
 * Transformers shell around its packed linears,
 * src/nanoquant/runtime/transformers_generation.py:84-114). */
int nq_add_rmsnorm(float* residual, const void* delta, int32_t delta_dtype, const void* weight,
                   int32_t weight_dtype, float eps, int64_t tokens, int64_t hidden, void* out,
                   int32_t out_dtype, void* stream);

/* Per-head RMSNorm of q and k (skipped when the weight is NULL), rotate-half
 * RoPE at positions position[0] + t, and the KV-cache append:
 *   q_out[t, h, :]              = rope(norm(q[t, h, :]))          (fp32)
 *   k_cache[g, position + t, :] = rope(norm(k[t, g, :]))          (cache_dtype)
 *   v_cache[g, position + t, :] = v[t, g, :]
 * head_dim is 64, 128 or 256; rows at or beyond max_positions are not
 * written. Replaces launch_decode_rope and launch_cache_prefix_update
 * (src/nanoquant/runtime/cuda_kernels.py:401-447,546-587,715-815) and the
 * q_norm / k_norm of the Qwen3 attention block. */
int nq_qk_norm_rope_cache(const float* q, const float* k, const float* v, int64_t tokens,
                          int32_t q_heads, int32_t kv_heads, int32_t head_dim, const void* q_norm,
                          const void* k_norm, int32_t norm_dtype, float eps, const float* cos_table,
                          const float* sin_table, const int32_t* position, int64_t max_positions,
                          float* q_out, void* k_cache, void* v_cache, int32_t cache_dtype,
                          void* stream);

/* Workspace bytes of nq_attention for `tokens` queries. */
int64_t nq_attention_workspace_bytes(int64_t tokens, int32_t q_heads, int32_t head_dim,
                                     int64_t max_positions);

/* Causal grouped-query attention: query t (at cache row position[0] + t)
 * attends cache rows [0, position[0] + t] of kv head h / (q_heads / kv_heads):
 *   out[t, h, :] = softmax(scaling * q[t, h, :] · K[g, 0..p, :]) · V[g, 0..p, :]
 * q fp32 [tokens, q_heads, head_dim]; out F32/F16/BF16 [tokens, q_heads *
 * head_dim]. Softmax in fp32. The sequence is split into 64-row blocks whose
 * partial results are merged in block order (deterministic). Replaces
 * launch_decode_attention (src/nanoquant/runtime/cuda_kernels.py:448-544),
 * generalised from its pinned one-kv-head, 64-row geometry. */
int nq_attention(const float* q, const void* k_cache, const void* v_cache, int32_t cache_dtype,
                 int64_t tokens, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                 const int32_t* position, int64_t max_positions, float scaling, void* out,
                 int32_t out_dtype, void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes of nq_decode_attention. */
int64_t nq_decode_attention_workspace_bytes(int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                            int32_t cache_dtype, int64_t max_positions);

/* One decode token: nq_qk_norm_rope_cache followed by nq_attention with
 * tokens == 1, as two kernels per layer when head_dim * cache element bytes
 * <= 256 and q_heads / kv_heads is 1, 2, 4 or 8 (pass 1: one workgroup per kv
 * head and 64-row cache block rotates its q heads, appends k/v at row
 * position[0] when the block holds it, and attends over the block; pass 2
 * merges the blocks' partial results), otherwise as the two calls. q, k, v are the fp32 projection outputs [q_heads * head_dim],
 * [kv_heads * head_dim] x2; out [q_heads * head_dim]. Replaces the pinned
 * one-token rope / cache update / attention sequence of the reference
 * (src/nanoquant/runtime/cuda_kernels.py:401-544,715-815). */
int nq_decode_attention(const float* q, const float* k, const float* v, int32_t q_heads, int32_t kv_heads,
                        int32_t head_dim, const void* q_norm, const void* k_norm, int32_t norm_dtype, float eps,
                        const float* cos_table, const float* sin_table, const int32_t* position,
                        int64_t max_positions, void* k_cache, void* v_cache, int32_t cache_dtype,
                        float scaling, void* out, int32_t out_dtype, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* Pass 1 of nq_decode_attention alone (the same arguments without the output;
 * the same workspace size): the partial results of every 64-row cache block
 * stay in the workspace, as fp32 (max, sum) pairs [q_heads][blocks][2]
 * followed by each block's output acc / sum in fp16 [q_heads][blocks][head_dim]
 * (a block's output is a weighted mean of V rows: values beyond the fp16 range
 * become infinite), blocks = ceil(max_positions / 64); a block past position[0]
 * holds the neutral partial (max -inf, sum 0, output 0), so a merge may run
 * over every block, weighting block s by sum_s * exp(max_s - max).
 * For a projection whose input merges them
 * (nq_linear_batch_fused with NQ_INPUT_ATTENTION). Only the one-pass form:
 * head_dim * cache element bytes <= 256 and q_heads / kv_heads 1, 2, 4 or 8,
 * otherwise NQ_ERR_UNSUPPORTED. No reference counterpart: the reference's
 * attention returns its output (src/nanoquant/runtime/cuda_kernels.py:715-815). */
int nq_decode_attention_partials(const float* q, const float* k, const float* v, int32_t q_heads,
                                 int32_t kv_heads, int32_t head_dim, const void* q_norm, const void* k_norm,
                                 int32_t norm_dtype, float eps, const float* cos_table, const float* sin_table,
                                 const int32_t* position, int64_t max_positions, void* k_cache, void* v_cache,
                                 int32_t cache_dtype, float scaling, void* workspace, int64_t workspace_bytes,
                                 void* stream);

/* out[i] = silu(gate[i]) * up[i], gate and up fp32, out F32/F16/BF16,
 * n % 8 == 0. Replaces the activation of Qwen3MLP.forward. */
int nq_silu_mul(const float* gate, const float* up, int64_t n, void* out, int32_t out_dtype,
                void* stream);

/* Workspace bytes of nq_output_projection (per-workgroup argmax partials). */
int64_t nq_output_projection_workspace_bytes(int64_t vocab, int64_t hidden);

/* logits[v] = Σ_i weight[v, i] * x[i] for one token: weight BF16 [vocab,
 * hidden] row-major, x F32/BF16 [hidden], fp32 accumulation, hidden % 8 == 0
 * and hidden <= 8192. Also leaves the per-workgroup (max, argmax) partials in
 * the workspace for nq_greedy_select. Replaces
 * launch_bfloat16_output_projection
 * (src/nanoquant/runtime/cuda_kernels.py:588-618,684-712). */
int nq_output_projection(const void* x, int32_t x_dtype, const void* weight, int64_t vocab,
                         int64_t hidden, float* logits, void* workspace, int64_t workspace_bytes,
                         void* stream);

/* Greedy token from the partials of the last nq_output_projection with the
 * same (vocab, hidden): the index of the largest logit, the lowest index on
 * ties (torch.argmax). Writes token_out[0]. When history and step are not
 * NULL, also history[*step] = token (only while *step < history_capacity)
 * and *step += 1; when position is not NULL, *position += 1. Replaces the
 * greedy branch of _sample_tokens
 * (src/nanoquant/runtime/generation.py:240-246). */
int nq_greedy_select(const void* workspace, int64_t vocab, int64_t hidden, int64_t* token_out,
                     int64_t* history, int64_t history_capacity, int32_t* step,
                     int32_t* position, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NQAMD_SHELL_H */
