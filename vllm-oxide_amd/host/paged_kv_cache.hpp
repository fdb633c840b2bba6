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
  void upload(const AttnMetadata& meta, hipStream_t stream);

  // Layer `layer`: append key/value [B, Hkv, D], then decode attention of
  // q [B, Hq, D] into out [B, Hq, D] (the order of models/qwen3.rs:199-208),
  // as one fused launch (paged_decode_attention_append).
  void run_layer(std::size_t layer, const void* q, const void* key, const void* value, void* out,
                 float softmax_scale, int32_t window_left, hipStream_t stream);

  std::size_t batch() const { return batch_; }

 private:
  void ensure(void** ptr, std::size_t* cap, std::size_t bytes);

  const PagedKVCache& cache_;
  std::size_t num_heads_;
  std::size_t batch_ = 0, max_blocks_ = 0, max_seqlen_k_ = 0;
  std::vector<uint32_t> h_cu_;
  std::vector<int32_t> h_table_;
  std::vector<int64_t> h_slots_;
  void* d_cu_ = nullptr;
  void* d_table_ = nullptr;
  void* d_slots_ = nullptr;
  void* d_ws_ = nullptr;
  std::size_t cap_cu_ = 0, cap_table_ = 0, cap_slots_ = 0, cap_ws_ = 0;
};

}  // namespace oxide::host
