/*
 * CPU oracle for the paged-KV hot path.  TEST INFRASTRUCTURE ONLY: it is the
 * checker that tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * compare the HIP library against.  The product library never links or calls
 * it, and nothing in the product falls back to it.
 *
 * Each function restates the reference algorithm it names (file:line under the
 * vllm-oxide tree) as plain loops.  How each one is pinned (golden vectors,
 * closed forms, independent brute force) is written next to it.
 */
#ifndef OXIDE_ORACLE_H
#define OXIDE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 16-bit float formats <-> fp32.  dtype: 0 = f16, 1 = bf16 (kernels.rs:97-104). */
float oracle_half_to_float(uint16_t h, int dtype);
uint16_t oracle_float_to_half(float f, int dtype); /* round to nearest even */

/* KvCacheManager::compute_slot_mapping, engine/kv_cache_manager.rs:115-135. */
void oracle_compute_slot_mapping(const int64_t* block_table, int64_t table_len,
                                 int64_t block_size, int64_t token_offset, int64_t num_tokens,
                                 int64_t* slot_mapping);

/* build_decode_metadata, attention/metadata.rs:20-47 (cu_seqlens_q/k have
 * batch + 1 entries; returns max_seqlen_k). */
int64_t oracle_build_decode_metadata(const uint32_t* context_lens, int64_t batch,
                                     uint32_t* cu_seqlens_q, uint32_t* cu_seqlens_k);

/* block_table_tensor, attention/flash_attn.rs:74-86: ragged rows (concatenated
 * in `flat`, row b has row_lens[b] entries) padded with 0 to [batch, max_len].
 * Returns max_len; `out` must hold batch * max_len entries. */
int64_t oracle_pad_block_table(const int32_t* flat, const int64_t* row_lens, int64_t batch,
                               int32_t* out);

/* reshape_and_cache kernel, kernels/reshape_and_cache.cu:6-28 (bitwise row
 * copy of esize-byte elements; slot == -1 skipped). */
void oracle_reshape_and_cache(const void* key, const void* value, void* key_cache,
                              void* value_cache, const int64_t* slot_mapping, int64_t num_tokens,
                              int64_t num_kv_heads, int64_t head_dim, int esize);

/* copy_blocks kernel, kernels/copy_blocks.cu:8-28 (pairs applied in order). */
void oracle_copy_blocks(void* key_cache, void* value_cache, const int64_t* block_mapping,
                        int64_t num_pairs, int64_t block_stride, int esize);

/* Prefix-hit gather (no reference counterpart): dst block i = cache block ids[i]. */
void oracle_gather_blocks(void* key_dst, void* value_dst, const void* key_cache,
                          const void* value_cache, const int32_t* block_ids, int64_t num_blocks,
                          int64_t block_stride, int esize);

/* Paged decode attention (the decode call of flash_attn_varlen_paged_windowed,
 * attention/flash_attn.rs:52-67): for each sequence b and query head h, keys
 * j in [lo, L_b), L_b = cu_seqlens_k[b+1] - cu_seqlens_k[b],
 * lo = window_left < 0 ? 0 : max(0, L_b - 1 - window_left), key j at cache row
 * block_table[b * max_blocks + j / block_size] * block_size + j % block_size,
 * kv head h / (num_heads / num_kv_heads);
 *   out[b,h,:] = sum_j softmax_j(scale * q.K_j) V_j.
 * Inputs are 16-bit (dtype 0/1).  Arithmetic in fp32 (use_f64 = 0: dot
 * products and sums accumulated in index order, two-pass softmax with expf) or
 * fp64 (use_f64 = 1).  Writes fp32 `out` [batch, num_heads, head_dim]; an
 * empty sequence gives zeros.  Parallel over (b, kv head) on `threads` OpenMP
 * threads (<= 0: OpenMP default). */
void oracle_paged_decode_attention(float* out, const uint16_t* q, const uint16_t* k_cache,
                                   const uint16_t* v_cache, const uint32_t* cu_seqlens_k,
                                   const int32_t* block_table, int64_t max_blocks, int64_t batch,
                                   int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                   int64_t block_size, int32_t window_left, float softmax_scale,
                                   int dtype, int use_f64, int threads);

/* Prefill attention: the general (seqlen_q >= 1) call of
 * flash_attn_varlen_paged_windowed with window_right = 0 (causal), and, with
 * block_table == NULL, flash_attn_varlen(..., causal = true) over contiguous
 * K/V (attention/flash_attn.rs:15-37).  Sequence b has Lq = cu_seqlens_q[b+1] -
 * cu_seqlens_q[b] queries (rows cu_seqlens_q[b] + i of q [total_q, Hq, D]) and
 * Lk = cu_seqlens_k[b+1] - cu_seqlens_k[b] keys.  Causal masks are aligned to
 * the bottom right, as in FlashAttention 2 for Lq != Lk: query i sees keys
 *   j <= hi = i + Lk - Lq   and, when window_left >= 0, j >= hi - window_left
 * (and 0 <= j < Lk).  A query with no visible key gives zeros.  Key j lives at
 * cache row block_table[b * max_blocks + j / block_size] * block_size +
 * j % block_size of [num_blocks, block_size, Hkv, D] (paged), or at row
 * cu_seqlens_k[b] + j of [total_k, Hkv, D] (block_table == NULL).  fp32 `out`
 * [total_q, Hq, D]; arithmetic as in oracle_paged_decode_attention. */
void oracle_prefill_attention(float* out, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const uint32_t* cu_seqlens_q, const uint32_t* cu_seqlens_k,
                              const int32_t* block_table, int64_t max_blocks, int64_t batch,
                              int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                              int64_t block_size, int32_t window_left, float softmax_scale,
                              int dtype, int use_f64, int threads);

/* RoPE cos/sin cache, layers/rope.rs:50-83: row t = [cos(t f_0..f_{R/2-1}),
 * sin(...)], f_i = 1 / base^(2i / R) in fp32, t f_i rounded to fp32. */
void oracle_rope_cos_sin_cache(float* cache, int64_t max_position, int64_t rotary_dim, float base);

/* The attention prologue of Qwen3Attention::forward (models/qwen3.rs:161-199):
 * split the merged qkv row [Hq*D | Hkv*D | Hkv*D] (row stride qkv_stride
 * elements), RMSNorm q and k per head (layers/rmsnorm.rs:52-87: fp32 upcast,
 * x / sqrt(mean(x^2) + eps), rounded to the dtype, times the weight, rounded;
 * skipped when the weight pointer is NULL), RoPE by positions[t]
 * (layers/rope.rs:133-163: y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin, each
 * product and sum rounded to fp32, result rounded to the dtype), then
 * reshape_and_cache of k and v at slot_mapping[t] (-1 skipped).  q_out
 * [T, Hq, D]; k_out [T, Hkv, D] optional.  The mean of squares is summed in
 * fp64 and rounded once to fp32 (the reference's reduction order is that of
 * its backend). */
void oracle_qk_norm_rope_and_cache(uint16_t* q_out, uint16_t* k_out, const uint16_t* qkv,
                                   int64_t qkv_stride, const uint16_t* q_norm_weight,
                                   const uint16_t* k_norm_weight, double eps,
                                   const float* cos_sin_cache, int64_t max_position,
                                   const int32_t* positions, uint16_t* key_cache,
                                   uint16_t* value_cache, const int64_t* slot_mapping,
                                   int64_t num_tokens, int64_t num_heads, int64_t num_kv_heads,
                                   int64_t head_dim, int dtype);

/* XXH64 (public xxHash spec, 64-bit variant) of `len` bytes with `seed`. */
uint64_t oracle_xxh64(const void* data, size_t len, uint64_t seed);

#ifdef __cplusplus
}
#endif

#endif /* OXIDE_ORACLE_H */
