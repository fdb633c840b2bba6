/*
 * oxide_paged_kv.h — C ABI of the MI355X (gfx950) paged-KV hot path.
 *
 * Every entry point takes plain device pointers, element counts and a
 * hipStream_t passed as `void*`.  Nothing here allocates device memory: the
 * caller owns every buffer, including the split-KV workspace of the decode
 * attention.  All launches are asynchronous on the given stream (NULL = the
 * default stream), which belongs to the calling thread's current HIP device
 * (the device whose CU count sizes the grids).  Entry points return void, as
 * the reference's do; argument
 * and launch errors are recorded per host thread and read back with
 * oxide_last_error() / oxide_error_string().
 *
 * Data layout (shared with the reference, crates/vllm-oxide/src/utils.rs:46-61
 * and crates/vllm-oxide/src/attention/mod.rs:78-85):
 *   physical buffer  [2, num_layers, num_blocks, block_size, num_kv_heads, head_dim]
 *   per-layer view   key_cache / value_cache = [num_blocks, block_size, num_kv_heads, head_dim]
 *   slot             block_id * block_size + offset_in_block  (row index of that view)
 *
 * dtype codes (crates/vllm-oxide/src/attention/kernels.rs:97-104):
 *   0 = f16, 1 = bf16, 2 = f32.
 */
#ifndef OXIDE_PAGED_KV_H
#define OXIDE_PAGED_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  OXIDE_DTYPE_F16 = 0,
  OXIDE_DTYPE_BF16 = 1,
  OXIDE_DTYPE_F32 = 2,
};

enum {
  OXIDE_OK = 0,
  OXIDE_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative count, bad stride */
  OXIDE_ERR_UNSUPPORTED_DTYPE = 2,
  OXIDE_ERR_UNSUPPORTED_SHAPE = 3, /* head_dim / group size / block size not built */
  OXIDE_ERR_WORKSPACE_TOO_SMALL = 4,
  OXIDE_ERR_SCRATCH_TOO_SMALL = 5, /* paged_decode_attention_noalloc: shape beyond its static scratch */
  OXIDE_ERR_HIP = 1000 /* OXIDE_ERR_HIP + hipError_t of a failed launch */
};

/*
 * KV append.  Replaces `extern "C" void reshape_and_cache(...)` of
 * crates/vllm-oxide/kernels/reshape_and_cache.cu:30-41 (Rust binding
 * crates/vllm-oxide/src/attention/kernels.rs:15-26); same symbol, same
 * parameters, `stream` is a hipStream_t.
 *
 * For token t in [0, num_tokens) with slot = slot_mapping[t] >= 0:
 *   key_cache  [slot * H*D + e] = key  [t * H*D + e]
 *   value_cache[slot * H*D + e] = value[t * H*D + e]    for e < H*D
 * where H = num_kv_heads, D = head_dim.  slot == -1 (the reference's sentinel,
 * kv_cache_manager.rs:128-131) leaves the cache untouched; any other negative
 * slot is treated the same way.  key/value are contiguous [T, H, D].  The copy
 * is bitwise, so it is bit-exact for every dtype.
 */
void reshape_and_cache(const void* key, const void* value, void* key_cache, void* value_cache,
                       const int64_t* slot_mapping, int64_t num_tokens, int64_t num_kv_heads,
                       int64_t head_dim, int dtype, void* stream);

/*
 * Block copy for prefix-cache copy-on-write.  Replaces `extern "C" void
 * copy_blocks(...)` of crates/vllm-oxide/kernels/copy_blocks.cu:30-38 (Rust
 * binding crates/vllm-oxide/src/attention/kernels.rs:28-36); same symbol and
 * parameters.
 *
 * block_mapping is a device int64 array [num_pairs, 2] of (src, dst) block
 * ids; block_stride is in ELEMENTS (block_size * num_kv_heads * head_dim,
 * kernels.rs:164-165).  For each pair, block dst of key_cache and of
 * value_cache becomes a bitwise copy of block src.  Precondition (as in the
 * reference, where it is unchecked): no dst block is also the src of another
 * pair in the same call.
 */
void copy_blocks(void* key_cache, void* value_cache, const int64_t* block_mapping,
                 int64_t num_pairs, int64_t block_stride, int dtype, void* stream);

/*
 * Prefix-hit block gather.  No reference counterpart (the reference never
 * reads prefix-hit blocks back from the paged cache,
 * crates/vllm-oxide/src/engine/mod.rs:172,195); it follows copy_blocks'
 * conventions.  For i < num_blocks:
 *   key_dst  [i * block_stride + e] = key_cache  [block_ids[i] * block_stride + e]
 *   value_dst[i * block_stride + e] = value_cache[block_ids[i] * block_stride + e]
 * so key_dst/value_dst come out as contiguous [num_blocks * block_size, H, D].
 * value_dst / value_cache may both be NULL to gather keys only.
 */
void gather_blocks(void* key_dst, void* value_dst, const void* key_cache, const void* value_cache,
                   const int32_t* block_ids, int64_t num_blocks, int64_t block_stride, int dtype,
                   void* stream);

/*
 * Paged decode attention with GQA, optional left sliding window and split-KV
 * (flash-decoding).  Replaces the decode call of
 * candle_flash_attn::flash_attn_varlen_paged_windowed made at
 * crates/vllm-oxide/src/attention/flash_attn.rs:52-67 (argument meanings in
 * research/prototype-candle-stack/src/main.rs:219-234).
 *
 *   out          [batch, num_heads, head_dim]        written (caller-allocated)
 *   q            [batch, num_heads, head_dim]        one query token per sequence
 *   k_cache      [num_blocks, page_block_size, num_kv_heads, head_dim]
 *   v_cache      same
 *   cu_seqlens_k uint32 [batch + 1], prefix sums of context lengths
 *                (build_decode_metadata, attention/metadata.rs:20-47)
 *   block_table  int32 [batch, max_blocks_per_seq], rows padded with 0
 *                (flash_attn.rs:74-86); only the first ceil(L_b / page_block_size)
 *                entries of row b are read
 *   num_blocks   blocks in k_cache / v_cache (dim 0 of the FA tensors); block
 *                ids outside [0, num_blocks) are clamped into range, so a bad
 *                table gives a wrong answer but never an out-of-bounds access
 *   max_seqlen_k max over b of L_b; sizes the split grid and the workspace.
 *                Lengths above it are clamped to it.
 *   window_left  -1 = unbounded (the reference passes None); w >= 0 attends to
 *                keys [max(0, L_b - 1 - w), L_b - 1]
 *   softmax_scale scale applied to q.k before the softmax (1/sqrt(head_dim) in
 *                the reference, models/qwen3.rs:204)
 *
 * Query head h reads kv head h / (num_heads / num_kv_heads).  A sequence with
 * L_b == 0 produces zeros.  Supported: dtype f16 or bf16, head_dim 64 or 128,
 * num_heads / num_kv_heads in 1..8 or 16 (Qwen3-14B has 5, Qwen2.5-7B 7),
 * page_block_size a positive
 * multiple of 16.  workspace must hold
 * paged_decode_attention_workspace_size(...) bytes for the same arguments (no
 * initialisation needed).  Calls that share a workspace must not overlap in
 * time.
 */
void paged_decode_attention(void* out, const void* q, const void* k_cache, const void* v_cache,
                            const uint32_t* cu_seqlens_k, const int32_t* block_table,
                            int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch,
                            int64_t num_heads,
                            int64_t num_kv_heads, int64_t head_dim, int64_t page_block_size,
                            int64_t max_seqlen_k, int32_t window_left, float softmax_scale,
                            void* workspace, size_t workspace_bytes, int dtype, void* stream);

/*
 * KV append fused into the decode attention launch: the same result as
 *   reshape_and_cache(key, value, k_cache, v_cache, slot_mapping, batch,
 *                     num_kv_heads, head_dim, dtype, stream);
 *   paged_decode_attention(out, q, k_cache, v_cache, ...);
 * (the append-then-attend order of models/qwen3.rs:199-208) in one launch.
 * key / value: [batch, num_kv_heads, head_dim], one new token per sequence;
 * slot_mapping[b] must be -1 or the cache slot of key L_b - 1 of sequence b,
 * which is what compute_slot_mapping gives at decode
 * (kv_cache_manager.rs:115-135, engine/mod.rs:250-257).  The workgroup that
 * attends to key L_b - 1 writes its kv head's slice of the new row and uses
 * it directly, so no extra ordering is needed.  Other arguments as for
 * paged_decode_attention (the same workspace size).
 */
void paged_decode_attention_append(void* out, const void* q, const void* key, const void* value,
                                   const int64_t* slot_mapping, void* k_cache, void* v_cache,
                                   const uint32_t* cu_seqlens_k, const int32_t* block_table,
                                   int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch,
                                   int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                   int64_t page_block_size, int64_t max_seqlen_k,
                                   int32_t window_left, float softmax_scale, void* workspace,
                                   size_t workspace_bytes, int dtype, void* stream);

/* Bytes of workspace paged_decode_attention needs for these arguments. */
size_t paged_decode_attention_workspace_size(int64_t batch, int64_t num_heads,
                                             int64_t num_kv_heads, int64_t head_dim,
                                             int64_t max_seqlen_k);

/* Tokens per KV split chosen for these arguments (128, 256, 512 or 1024) when the
 * split grid is chosen; -1 when the wave-level stream pass is chosen (kv
 * heads dividing 8, at least ~1024 keys per stream range -- batch *
 * max_seqlen_k >= 1024 * CUs * 8 / num_kv_heads -- and at least 16 sequences
 * or 4096 keys per range; it splits each head's keys
 * evenly over CUs * 8 / num_kv_heads ranges, one per wave); 0 when the
 * balanced persistent pass is chosen (other kv head counts at long contexts:
 * batch * max_seqlen_k * num_kv_heads >= 16384 positions per resident
 * workgroup). */
int64_t paged_decode_attention_split_tokens(int64_t batch, int64_t num_kv_heads,
                                            int64_t max_seqlen_k);

/*
 * paged_decode_attention (key, value and slot_mapping all NULL) or
 * paged_decode_attention_append (all three given) with the first pass chosen
 * by the caller instead of by shape.  No counterpart in the reference; for
 * tuning and tests.  The choice is an argument of this call only: the library
 * keeps no state between calls that changes what a call computes.  path: 0 = by shape (as the plain entries),
 * 1 = the split grid, 2 = the persistent pass, 3 = the stream pass where the
 * kv heads divide 8 (else the persistent pass), 4 = the row pass where the shape
 * allows it (head_dim 128, 8 kv heads, 32 query heads, power-of-two pages, at
 * most 1024 sequences; else as 3); anything else is
 * OXIDE_ERR_INVALID_ARGUMENT.  Results agree within rounding; the workspace
 * size is the same for every path.
 */
void paged_decode_attention_path(int path, void* out, const void* q, const void* key, const void* value,
                                 const int64_t* slot_mapping, void* k_cache, void* v_cache,
                                 const uint32_t* cu_seqlens_k, const int32_t* block_table,
                                 int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch,
                                 int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                 int64_t page_block_size, int64_t max_seqlen_k, int32_t window_left,
                                 float softmax_scale, void* workspace, size_t workspace_bytes, int dtype,
                                 void* stream);

/* paged_decode_attention_split_tokens for the first pass that
 * paged_decode_attention_path(path, ...) runs on these arguments (path 0 =
 * by shape; codes outside 0..3 read as 0).  No reference counterpart. */
int64_t paged_decode_attention_path_split_tokens(int path, int64_t batch, int64_t num_kv_heads,
                                                 int64_t max_seqlen_k);

/*
 * Paged decode attention (key, value and slot_mapping all NULL) or the fused
 * append + attention (all three given) of a batch whose block-table rows share
 * their leading entries -- a common prompt prefix cached once (the BlockPool's
 * prefix sharing) -- computed as a cascade: the shared keys are attended once for
 * every sequence (matrix cores, all (sequence, query head) rows against each
 * shared K/V tile), the remaining keys per sequence by the decode stream pass, and
 * the two merged with log-sum-exp weights.  Same results as
 * paged_decode_attention(_append) within rounding; no reference counterpart (the
 * reference reads the shared blocks once per sequence).
 * shared_blocks_hint: an upper bound on the leading entries shared by every row
 * (0 = no cascade: the plain entries run; so do batches where the cascade would
 * not pay, see paged_decode_attention_shared_prefix_plan).  The kernels find the actual count on
 * the device (identical block ids in every row, and at most (L_b - 1) / block_size
 * for every sequence), so a wrong hint costs time, never correctness.  Shapes the
 * stream pass does not take (kv heads not dividing 8, more than 4096 sequences)
 * run the plain entries.  workspace: paged_decode_attention_shared_prefix_workspace_size
 * bytes.  Other arguments as for paged_decode_attention_append.
 * When the per-sequence part is long enough to hide it, the shared-key pass runs
 * beside the stream pass on a side stream the library keeps per host thread and
 * device (created on the thread's first such call, default priority), forked from
 * `stream` and joined back into it with two events: all work is still ordered
 * after what `stream` held before the call and before what it receives after, and
 * under HIP graph capture the fork and join become graph edges (one thread
 * capturing two graphs at once, each with an overlapped call, would tie both to
 * the same side stream: end one capture before the next call of the other).
 */
void paged_decode_attention_shared_prefix(void* out, const void* q, const void* key, const void* value,
                                          const int64_t* slot_mapping, void* k_cache, void* v_cache,
                                          const uint32_t* cu_seqlens_k, const int32_t* block_table,
                                          int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch,
                                          int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                          int64_t page_block_size, int64_t max_seqlen_k, int32_t window_left,
                                          float softmax_scale, int64_t shared_blocks_hint, void* workspace,
                                          size_t workspace_bytes, int dtype, void* stream);

/*
 * paged_decode_attention_shared_prefix with its form chosen by the caller instead
 * of by shape.  No counterpart in the reference; for tuning and tests.  mode:
 * 0 = by shape (as paged_decode_attention_shared_prefix), 1 = the cascade with
 * its two passes one after the other, 2 = the cascade with the shared-key pass
 * beside the per-sequence pass on the side stream, 3 = the plain entries; other
 * values are OXIDE_ERR_INVALID_ARGUMENT.  Shapes the cascade does not take run
 * the plain entries whatever the mode.  Results agree within rounding; the
 * workspace size is the same for every mode.
 */
void paged_decode_attention_shared_prefix_mode(int mode, void* out, const void* q, const void* key,
                                               const void* value, const int64_t* slot_mapping, void* k_cache,
                                               void* v_cache, const uint32_t* cu_seqlens_k,
                                               const int32_t* block_table, int64_t max_blocks_per_seq,
                                               int64_t num_blocks, int64_t batch, int64_t num_heads,
                                               int64_t num_kv_heads, int64_t head_dim, int64_t page_block_size,
                                               int64_t max_seqlen_k, int32_t window_left, float softmax_scale,
                                               int64_t shared_blocks_hint, void* workspace, size_t workspace_bytes,
                                               int dtype, void* stream);

/* The form paged_decode_attention_shared_prefix (mode 0) takes on these
 * arguments: 1, 2 or 3 as for paged_decode_attention_shared_prefix_mode.  The
 * cascade runs only where the K/V bytes it saves (the shared keys read once
 * instead of once per sequence) outweigh its extra pass; no reference
 * counterpart. */
int paged_decode_attention_shared_prefix_plan(int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                                              int64_t head_dim, int64_t page_block_size, int64_t max_seqlen_k,
                                              int64_t shared_blocks_hint);

/* Bytes of workspace paged_decode_attention_shared_prefix needs (at least
 * paged_decode_attention_workspace_size, so the fallback fits too). */
size_t paged_decode_attention_shared_prefix_workspace_size(int64_t batch, int64_t num_heads,
                                                           int64_t num_kv_heads, int64_t head_dim,
                                                           int64_t page_block_size, int64_t max_seqlen_k,
                                                           int64_t shared_blocks_hint);

/* The first pass paged_decode_attention_path(path, ...) runs on these arguments
 * (path 0 = by shape, as the plain entries; codes outside 0..4 read as 0): the
 * split size (> 0) for the split grid, 0 for the persistent pass, -1 for the
 * stream pass, -2 for the row pass.  Unlike the two queries above it knows the
 * query heads, head size and page size, which the row pass depends on.  No
 * reference counterpart. */
int64_t paged_decode_attention_pass1(int path, int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                                     int64_t head_dim, int64_t page_block_size, int64_t max_seqlen_k);

/*
 * Prefill attention over the paged cache.  Replaces the general (seqlen_q >= 1)
 * call of candle_flash_attn::flash_attn_varlen_paged_windowed
 * (crates/vllm-oxide/src/attention/flash_attn.rs:52-67) with window_right =
 * Some(0), i.e. causal.  The prompt's K/V are appended first
 * (reshape_and_cache with the prefill slot mapping, engine/mod.rs:186-191,
 * models/qwen3.rs:199); keys already in the cache (a prefix hit, earlier
 * chunks) are the first Lk - Lq keys of the sequence and need no gather.
 *
 *   out          [total_q, num_heads, head_dim]  written (caller-allocated)
 *   q            [total_q, num_heads, head_dim]  rows cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1
 *   cu_seqlens_q uint32 [batch + 1], prefix sums of query counts Lq_b
 *                (build_prefill_metadata, attention/metadata.rs:49-80)
 *   cu_seqlens_k uint32 [batch + 1], prefix sums of key counts Lk_b (the
 *                whole context, new tokens included)
 *   block_table, num_blocks, page_block_size, k_cache, v_cache: as for
 *                paged_decode_attention
 *   max_seqlen_q / max_seqlen_k  maxima of Lq_b / Lk_b (size the grid; larger
 *                lengths are clamped to them)
 *   window_left  -1 = none; w >= 0 limits query i to keys >= hi - w
 *
 * Masks are aligned to the bottom right, as in FlashAttention 2: query i of
 * sequence b sees keys j with j <= hi = i + Lk_b - Lq_b (and j >= hi - w).
 * A query that sees no key (Lk_b < Lq_b) gets zeros.  Supported: f16/bf16,
 * head_dim 64 or 128, num_heads / num_kv_heads <= 128, any positive
 * page_block_size.  No workspace.
 */
void paged_prefill_attention(void* out, const void* q, const void* k_cache, const void* v_cache,
                             const uint32_t* cu_seqlens_q, const uint32_t* cu_seqlens_k,
                             const int32_t* block_table, int64_t max_blocks_per_seq,
                             int64_t num_blocks, int64_t batch, int64_t num_heads,
                             int64_t num_kv_heads, int64_t head_dim, int64_t page_block_size,
                             int64_t max_seqlen_q, int64_t max_seqlen_k, int32_t window_left,
                             float softmax_scale, int dtype, void* stream);

/*
 * The same attention over contiguous K/V.  Replaces
 * candle_flash_attn::flash_attn_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k,
 * max_seqlen_q, max_seqlen_k, softmax_scale, causal = true) of prefill_attn,
 * crates/vllm-oxide/src/attention/flash_attn.rs:15-37.  k / v are
 * [total_k, num_kv_heads, head_dim]; key j of sequence b is row
 * cu_seqlens_k[b] + j (rows >= total_k are clamped).  Other arguments and the
 * mask as for paged_prefill_attention.
 */
void varlen_prefill_attention(void* out, const void* q, const void* k, const void* v,
                              const uint32_t* cu_seqlens_q, const uint32_t* cu_seqlens_k,
                              int64_t total_k, int64_t batch, int64_t num_heads,
                              int64_t num_kv_heads, int64_t head_dim, int64_t max_seqlen_q,
                              int64_t max_seqlen_k, int32_t window_left, float softmax_scale,
                              int dtype, void* stream);

/*
 * The attention prologue fused with the KV append.  Replaces, per token t, the
 * chain of Qwen3Attention::forward (crates/vllm-oxide/src/models/qwen3.rs:161-199):
 * split of the merged qkv row, q_norm / k_norm (layers/rmsnorm.rs:52-87),
 * rotary_emb.forward (layers/rope.rs:133-163) and
 * PagedKVCache::reshape_and_cache(k, v, slot_mapping) (qwen3.rs:199).
 *
 *   q_out          [T, num_heads, head_dim]      written: normed + rotated q
 *   k_out          [T, num_kv_heads, head_dim]   optional (NULL = not written)
 *   qkv            [T, qkv_row_stride], row = q (Hq*D) | k (Hkv*D) | v (Hkv*D)
 *   q_norm_weight, k_norm_weight   [head_dim] in the dtype, or NULL: no norm
 *                  (Qwen3 with attention bias has none, qwen3.rs:118-136)
 *   eps            rms_norm_eps
 *   cos_sin_cache  fp32 [max_position, head_dim] (oxide_rope_cos_sin_cache);
 *                  positions outside [0, max_position) are clamped into it
 *   positions      int32 [T]
 *   key_cache, value_cache, slot_mapping   as for reshape_and_cache; with
 *                  slot_mapping == NULL nothing is appended
 *
 * Per head: x -> round(round(x / sqrt(mean(x^2) + eps)) * w), then
 * y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin (halves x1 = x[:D/2],
 * x2 = x[D/2:]), each product and sum rounded to fp32, y rounded to the dtype.
 * v is copied bitwise.  Supported: f16/bf16, head_dim 64 or 128.
 */
void qk_norm_rope_and_cache(void* q_out, void* k_out, const void* qkv, int64_t qkv_row_stride,
                            const void* q_norm_weight, const void* k_norm_weight, double eps,
                            const float* cos_sin_cache, int64_t max_position,
                            const int32_t* positions, void* key_cache, void* value_cache,
                            const int64_t* slot_mapping, int64_t num_tokens, int64_t num_heads,
                            int64_t num_kv_heads, int64_t head_dim, int dtype, void* stream);

/*
 * Host helper: fills `cache` (host memory, max_position * rotary_dim floats)
 * with RotaryEmbedding's cos_sin_cache (crates/vllm-oxide/src/layers/rope.rs:50-83):
 * row t = [cos(t f_i) | sin(t f_i)], f_i = 1 / base^(2i / rotary_dim), fp32.
 * Returns OXIDE_OK or OXIDE_ERR_INVALID_ARGUMENT.
 */
int oxide_rope_cos_sin_cache(float* cache, int64_t max_position, int64_t rotary_dim, float base);

/*
 * Decode metadata on the device (the reference builds it on the host in every
 * layer: crates/vllm-oxide/src/engine/mod.rs:247-267, metadata.rs:20-47,
 * kv_cache_manager.rs:115-135).  From context_lens (uint32 [batch], the new
 * token included) and the 0-padded int32 block table [batch, max_blocks_per_seq]:
 *   cu_seqlens_k[0] = 0, cu_seqlens_k[b+1] = cu_seqlens_k[b] + context_lens[b]
 *   slot_mapping[b] = block_table[b][(L-1)/block_size] * block_size + (L-1) % block_size,
 *                     L = context_lens[b]; -1 when L == 0 or (L-1)/block_size >= max_blocks_per_seq.
 * One small launch; batch <= 65535.
 */
void build_decode_metadata_device(const uint32_t* context_lens, const int32_t* block_table,
                                  int64_t max_blocks_per_seq, int64_t batch, int64_t block_size,
                                  uint32_t* cu_seqlens_k, int64_t* slot_mapping, void* stream);

/*
 * paged_decode_attention_append (key, value, slot_mapping given) or
 * paged_decode_attention (all three NULL) without a workspace argument: the
 * split-KV partials live in a static device array of 48 MiB that each device
 * holds from the library's load until the process ends.  No counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops that forbid allocation).  The call allocates
 * nothing and its kernels need no cleared memory (every partial is written
 * before it is read).  A shape whose first pass needs more than the array
 * (its partial rows, their log-sum-exps and, windowed, the attended-key
 * prefix sums) is rejected with OXIDE_ERR_SCRATCH_TOO_SMALL and launches
 * nothing.  The stream pass (the shape policy's choice for batches of 16 or
 * more sequences with long contexts) needs 2 rows per wave slot and query of the
 * group (2 x CUs x 16 x G rows): Qwen3 shapes with up to 16 query heads per kv
 * head at head_dim 128 fit at any batch it takes.  The split grid (smaller
 * batches) needs a row per (sequence, query head, split): with
 * rows = batch x num_heads x ceil(max_seqlen_k / split), split =
 * paged_decode_attention_split_tokens(...) when it returns > 0, the call fits
 * when round_up(rows x head_dim x 4, 256) + round_up(rows x 4, 256) <= 48 MiB
 * (at 1024-key splits, head_dim 128: rows <= 97,541, e.g. 15 sequences of 64k
 * keys at 128 query heads do not fit).  A caller that captures graphs can check
 * a shape with that bound before capture.  The first call on a device resolves
 * the array's address; it may itself be made under graph capture (the query
 * enqueues nothing).  Every call on one device shares
 * that device's array: calls that overlap in time on one device (two streams,
 * two threads) race and give wrong results; calls ordered on one stream do not.
 * Other arguments and results as for paged_decode_attention_append.
 */
void paged_decode_attention_noalloc(void* out, const void* q, const void* key, const void* value,
                                    const int64_t* slot_mapping, void* k_cache, void* v_cache,
                                    const uint32_t* cu_seqlens_k, const int32_t* block_table,
                                    int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch,
                                    int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                    int64_t page_block_size, int64_t max_seqlen_k, int32_t window_left,
                                    float softmax_scale, int dtype, void* stream);

/* Error state of the calling host thread: the first error since the last
 * oxide_clear_error(), or OXIDE_OK. */
int oxide_last_error(void);
void oxide_clear_error(void);
const char* oxide_error_string(int code);

#ifdef __cplusplus
}
#endif

#endif /* OXIDE_PAGED_KV_H */
