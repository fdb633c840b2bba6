// Physical paged KV cache on one GPU and the per-step decode driver.
//
// PagedKVCache mirrors crates/vllm-oxide/src/attention/mod.rs:48-112: one
// zero-filled buffer [2, L, NB, BS, Hkv, D] with per-layer K/V views and
// reshape_and_cache.  DecodeStep holds the device copies of one step's
// AttnMetadata (cu_seqlens_k, padded block table, slot mapping) and the
// split-KV workspace; it uploads them once per step and every layer reuses
// them, where the reference re-uploads them in every layer
// (models/qwen3.rs:189-193, attention/flash_attn.rs:46-50).
#pragma once

#include <hip/hip_runtime.h>

#include "oxide_host.hpp"
#include "oxide_paged_kv.h"

namespace oxide::host {

class HipError : public std::runtime_error {
 public:
  explicit HipError(const std::string& m) : std::runtime_error(m) {}
};

class PagedKVCache {
 public:
  PagedKVCache(std::size_t num_layers, std::size_t num_blocks, std::size_t block_size,
               std::size_t num_kv_heads, std::size_t head_dim, int dtype);
  ~PagedKVCache();
  PagedKVCache(const PagedKVCache&) = delete;
  PagedKVCache& operator=(const PagedKVCache&) = delete;

  // Per-layer views [num_blocks, block_size, num_kv_heads, head_dim].
  void* k_cache(std::size_t layer) const;
  void* v_cache(std::size_t layer) const;
  std::array<std::size_t, 6> buffer_shape() const;
  std::size_t num_blocks() const { return num_blocks_; }
  std::size_t block_size() const { return block_size_; }
  std::size_t num_kv_heads() const { return num_kv_heads_; }
  std::size_t head_dim() const { return head_dim_; }
  int dtype() const { return dtype_; }
  std::size_t elem_bytes() const;

  // key/value: device [num_tokens, Hkv, D]; slot_mapping: device int64 [num_tokens].
  void reshape_and_cache(std::size_t layer, const void* key, const void* value,
                         const int64_t* slot_mapping, std::size_t num_tokens,
                         hipStream_t stream) const;
  // block_mapping: device int64 [num_pairs, 2] (src, dst), applied to one layer.
  void copy_blocks(std::size_t layer, const int64_t* block_mapping, std::size_t num_pairs,
                   hipStream_t stream) const;
  // Copy-on-write copies of a step (host (src, dst) block pairs, e.g. from
  // KvCacheManager::may_append_cow) in every layer, K and V, with one launch:
  // block b of layer l is block l * num_blocks + b of the buffer's K (V) half.
  void copy_blocks_all_layers(const std::vector<std::pair<std::size_t, std::size_t>>& pairs,
                              hipStream_t stream);

 private:
  std::size_t num_layers_, num_blocks_, block_size_, num_kv_heads_, head_dim_;
  int dtype_;
  void* buffer_ = nullptr;
  std::vector<int64_t> h_map_;  // staging of copy_blocks_all_layers
  void* d_map_ = nullptr;
  std::size_t cap_map_ = 0;
};

class DecodeStep {
 public:
  DecodeStep(const PagedKVCache& cache, std::size_t num_heads);
  ~DecodeStep();
  DecodeStep(const DecodeStep&) = delete;
  DecodeStep& operator=(const DecodeStep&) = delete;

  // Uploads cu_seqlens_k, the 0-padded block table and the slot mapping of
  // this step (asynchronous on `stream`; the host copy stays alive inside).
  // Also counts the leading block-table entries every row holds in common: the
  // prefix blocks the BlockPool handed to every sequence (block_pool.rs:133-142
  // sharing), the hint of the cascaded attention entry.
  void upload(const AttnMetadata& meta, hipStream_t stream);

  // Layer `layer`: append key/value [B, Hkv, D], then decode attention of
  // q [B, Hq, D] into out [B, Hq, D] (the order of models/qwen3.rs:199-208),
  // as one fused launch (paged_decode_attention_append; with a shared prefix,
  // paged_decode_attention_shared_prefix, which attends the shared blocks once
  // for the batch where that pays).
  void run_layer(std::size_t layer, const void* q, const void* key, const void* value, void* out,
                 float softmax_scale, int32_t window_left, hipStream_t stream);

  std::size_t batch() const { return batch_; }
  // Leading block-table entries common to every row of the uploaded step (0 for
  // a batch of one).
  std::size_t shared_blocks() const { return shared_blocks_; }

 private:
  void ensure(void** ptr, std::size_t* cap, std::size_t bytes);

  const PagedKVCache& cache_;
  std::size_t num_heads_;
  std::size_t batch_ = 0, max_blocks_ = 0, max_seqlen_k_ = 0, shared_blocks_ = 0;
  std::vector<uint32_t> h_cu_;
  std::vector<int32_t> h_table_;
  std::vector<int64_t> h_slots_;
  void* d_cu_ = nullptr;
  void* d_table_ = nullptr;
  void* d_slots_ = nullptr;
  void* d_ws_ = nullptr;
  std::size_t cap_cu_ = 0, cap_table_ = 0, cap_slots_ = 0, cap_ws_ = 0;
};

// The prefill step on the paged cache: per step, upload cu_seqlens_q / _k, the
// padded block table, the slot mapping and the positions once; per layer, run
// the attention prologue (q/k norm + RoPE + append of the prompt's K/V,
// qwen3.rs:161-199) and paged prefill attention over every key of the
// sequence, cached prefix included.  The reference's prefill reads only the
// projection K/V (flash_attn_varlen, engine/mod.rs:172,195) and so cannot use
// a prefix hit; here the prefix keys are simply the first Lk - Lq keys.
class PrefillStep {
 public:
  PrefillStep(const PagedKVCache& cache, std::size_t num_heads);
  ~PrefillStep();
  PrefillStep(const PrefillStep&) = delete;
  PrefillStep& operator=(const PrefillStep&) = delete;

  // meta from build_prefill_metadata (its block_table is not used);
  // block_table: each sequence's block ids (covering its kv length);
  // positions: the position of each scheduled token (engine/mod.rs:176-183).
  void upload(const AttnMetadata& meta, const std::vector<std::vector<int32_t>>& block_table,
              const std::vector<int32_t>& positions, hipStream_t stream);

  // Layer `layer`: qkv [T, (Hq + 2 Hkv) D] -> q_scratch [T, Hq, D] (normed,
  // rotated), K/V appended at the slot mapping, out [T, Hq, D].  Norm weights
  // may be null (no q/k norm); cos_sin is the fp32 [max_position, D] table.
  void run_layer(std::size_t layer, const void* qkv, const void* q_norm_weight, const void* k_norm_weight,
                 double eps, const float* cos_sin, std::size_t max_position, void* q_scratch, void* out,
                 float softmax_scale, int32_t window_left, hipStream_t stream);

  std::size_t num_tokens() const { return num_tokens_; }

 private:
  const PagedKVCache& cache_;
  std::size_t num_heads_;
  std::size_t batch_ = 0, num_tokens_ = 0, max_blocks_ = 0, max_seqlen_q_ = 0, max_seqlen_k_ = 0;
  std::vector<uint32_t> h_cuq_, h_cuk_;
  std::vector<int32_t> h_table_, h_pos_;
  std::vector<int64_t> h_slots_;
  void* d_buf_ = nullptr;  // cu_q | cu_k | table | positions | slots, 256-byte aligned parts
  std::size_t cap_ = 0;
  std::size_t off_cuk_ = 0, off_table_ = 0, off_pos_ = 0, off_slots_ = 0;
};

}  // namespace oxide::host
