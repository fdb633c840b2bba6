// PagedKVCache and DecodeStep over the C ABI (see paged_kv_cache.hpp).
#include "paged_kv_cache.hpp"

#include <algorithm>
#include <unordered_set>

namespace oxide::host {

namespace {
void check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw HipError(std::string(what) + ": " + hipGetErrorString(e));
}
void check_lib(const char* what) {
  const int code = oxide_last_error();
  if (code != OXIDE_OK) {
    oxide_clear_error();
    throw HipError(std::string(what) + ": " + oxide_error_string(code));
  }
}
}  // namespace

PagedKVCache::PagedKVCache(std::size_t num_layers, std::size_t num_blocks, std::size_t block_size,
                           std::size_t num_kv_heads, std::size_t head_dim, int dtype)
    : num_layers_(num_layers),
      num_blocks_(num_blocks),
      block_size_(block_size),
      num_kv_heads_(num_kv_heads),
      head_dim_(head_dim),
      dtype_(dtype) {
  if (elem_bytes() == 0) throw std::invalid_argument("unsupported KV cache dtype");
  const auto s = buffer_shape();
  std::size_t bytes = elem_bytes();
  for (std::size_t d : s) bytes *= d;
  check(hipMalloc(&buffer_, std::max<std::size_t>(bytes, 1)), "hipMalloc(PagedKVCache)");
  check(hipMemset(buffer_, 0, bytes), "hipMemset(PagedKVCache)");  // Tensor::zeros, mod.rs:68
}

PagedKVCache::~PagedKVCache() {
  if (buffer_) (void)hipFree(buffer_);
  if (d_map_) (void)hipFree(d_map_);
}

std::size_t PagedKVCache::elem_bytes() const {
  return dtype_ == OXIDE_DTYPE_F32 ? 4 : (dtype_ == OXIDE_DTYPE_F16 || dtype_ == OXIDE_DTYPE_BF16 ? 2 : 0);
}

std::array<std::size_t, 6> PagedKVCache::buffer_shape() const {
  return kv_cache_layout_shape(num_layers_, num_blocks_, block_size_, num_kv_heads_, head_dim_);
}

void* PagedKVCache::k_cache(std::size_t layer) const {
  if (layer >= num_layers_) throw std::out_of_range("layer");
  const std::size_t view = num_blocks_ * block_size_ * num_kv_heads_ * head_dim_ * elem_bytes();
  return static_cast<char*>(buffer_) + layer * view;
}

void* PagedKVCache::v_cache(std::size_t layer) const {
  if (layer >= num_layers_) throw std::out_of_range("layer");
  const std::size_t view = num_blocks_ * block_size_ * num_kv_heads_ * head_dim_ * elem_bytes();
  return static_cast<char*>(buffer_) + (num_layers_ + layer) * view;
}

void PagedKVCache::reshape_and_cache(std::size_t layer, const void* key, const void* value,
                                     const int64_t* slot_mapping, std::size_t num_tokens,
                                     hipStream_t stream) const {
  ::reshape_and_cache(key, value, k_cache(layer), v_cache(layer), slot_mapping,
                      static_cast<int64_t>(num_tokens), static_cast<int64_t>(num_kv_heads_),
                      static_cast<int64_t>(head_dim_), dtype_, stream);
  check_lib("reshape_and_cache");
}

void PagedKVCache::copy_blocks(std::size_t layer, const int64_t* block_mapping,
                               std::size_t num_pairs, hipStream_t stream) const {
  ::copy_blocks(k_cache(layer), v_cache(layer), block_mapping, static_cast<int64_t>(num_pairs),
                static_cast<int64_t>(block_size_ * num_kv_heads_ * head_dim_), dtype_, stream);
  check_lib("copy_blocks");
}

void PagedKVCache::copy_blocks_all_layers(const std::vector<std::pair<std::size_t, std::size_t>>& pairs,
                                          hipStream_t stream) {
  if (pairs.empty()) return;
  // The copy kernel runs every pair at once: a destination that is also a
  // source, or written twice, would race (copy_blocks.cu:20-27 leaves this
  // unchecked).  The pairs are on the host here, so check them.
  std::unordered_set<std::size_t> srcs, dsts;
  for (const auto& pr : pairs) {
    if (pr.first >= num_blocks_ || pr.second >= num_blocks_) throw std::out_of_range("block id");
    srcs.insert(pr.first);
    if (!dsts.insert(pr.second).second) throw std::invalid_argument("copy_blocks: a block is written twice");
  }
  for (std::size_t d : dsts)
    if (srcs.count(d)) throw std::invalid_argument("copy_blocks: a destination block is also a source");
  // The previous call's upload may still read the staging copy.
  check(hipStreamSynchronize(stream), "hipStreamSynchronize");
  h_map_.clear();
  for (std::size_t l = 0; l < num_layers_; ++l)
    for (const auto& pr : pairs) {
      h_map_.push_back(static_cast<int64_t>(l * num_blocks_ + pr.first));
      h_map_.push_back(static_cast<int64_t>(l * num_blocks_ + pr.second));
    }
  const std::size_t bytes = h_map_.size() * sizeof(int64_t);
  if (bytes > cap_map_) {
    if (d_map_) check(hipFree(d_map_), "hipFree");
    d_map_ = nullptr;
    check(hipMalloc(&d_map_, bytes), "hipMalloc(copy map)");
    cap_map_ = bytes;
  }
  check(hipMemcpyAsync(d_map_, h_map_.data(), bytes, hipMemcpyHostToDevice, stream), "upload copy map");
  ::copy_blocks(k_cache(0), v_cache(0), static_cast<const int64_t*>(d_map_),
                static_cast<int64_t>(h_map_.size() / 2),
                static_cast<int64_t>(block_size_ * num_kv_heads_ * head_dim_), dtype_, stream);
  check_lib("copy_blocks (all layers)");
}

DecodeStep::DecodeStep(const PagedKVCache& cache, std::size_t num_heads)
    : cache_(cache), num_heads_(num_heads) {}

DecodeStep::~DecodeStep() {
  for (void* p : {d_cu_, d_table_, d_slots_, d_ws_})
    if (p) (void)hipFree(p);
}

void DecodeStep::ensure(void** ptr, std::size_t* cap, std::size_t bytes) {
  if (bytes <= *cap) return;
  if (*ptr) check(hipFree(*ptr), "hipFree");
  *ptr = nullptr;
  check(hipMalloc(ptr, bytes), "hipMalloc(DecodeStep)");
  *cap = bytes;
}

void DecodeStep::upload(const AttnMetadata& meta, hipStream_t stream) {
  if (meta.is_prefill) throw std::invalid_argument("DecodeStep needs decode metadata");
  batch_ = meta.cu_seqlens_k.empty() ? 0 : meta.cu_seqlens_k.size() - 1;
  if (batch_ == 0) return;
  const PaddedTable t = pad_block_table(meta.block_table);
  max_blocks_ = t.width;
  max_seqlen_k_ = meta.max_seqlen_k;
  // Synchronise before overwriting the staging copies a previous async upload may still read.
  check(hipStreamSynchronize(stream), "hipStreamSynchronize");
  h_cu_ = meta.cu_seqlens_k;
  h_table_ = t.data;
  h_slots_ = meta.slot_mapping;
  ensure(&d_cu_, &cap_cu_, h_cu_.size() * sizeof(uint32_t));
  ensure(&d_table_, &cap_table_, std::max<std::size_t>(h_table_.size(), 1) * sizeof(int32_t));
  ensure(&d_slots_, &cap_slots_, std::max<std::size_t>(h_slots_.size(), 1) * sizeof(int64_t));
  check(hipMemcpyAsync(d_cu_, h_cu_.data(), h_cu_.size() * sizeof(uint32_t), hipMemcpyHostToDevice,
                       stream), "upload cu_seqlens_k");
  check(hipMemcpyAsync(d_table_, h_table_.data(), h_table_.size() * sizeof(int32_t),
                       hipMemcpyHostToDevice, stream), "upload block_table");
  check(hipMemcpyAsync(d_slots_, h_slots_.data(), h_slots_.size() * sizeof(int64_t),
                       hipMemcpyHostToDevice, stream), "upload slot_mapping");
  // Leading entries every row holds (bounded by the shortest row).
  shared_blocks_ = 0;
  if (batch_ > 1) {
    std::size_t n = meta.block_table[0].size();
    for (const auto& row : meta.block_table) n = std::min(n, row.size());
    while (shared_blocks_ < n) {
      const int32_t id = meta.block_table[0][shared_blocks_];
      bool same = true;
      for (const auto& row : meta.block_table) same = same && row[shared_blocks_] == id;
      if (!same) break;
      ++shared_blocks_;
    }
  }
  const std::size_t ws =
      shared_blocks_ > 0
          ? paged_decode_attention_shared_prefix_workspace_size(
                static_cast<int64_t>(batch_), static_cast<int64_t>(num_heads_),
                static_cast<int64_t>(cache_.num_kv_heads()), static_cast<int64_t>(cache_.head_dim()),
                static_cast<int64_t>(cache_.block_size()), static_cast<int64_t>(max_seqlen_k_),
                static_cast<int64_t>(shared_blocks_))
          : paged_decode_attention_workspace_size(
                static_cast<int64_t>(batch_), static_cast<int64_t>(num_heads_),
                static_cast<int64_t>(cache_.num_kv_heads()), static_cast<int64_t>(cache_.head_dim()),
                static_cast<int64_t>(max_seqlen_k_));
  ensure(&d_ws_, &cap_ws_, std::max<std::size_t>(ws, 1));
}

void DecodeStep::run_layer(std::size_t layer, const void* q, const void* key, const void* value,
                           void* out, float softmax_scale, int32_t window_left,
                           hipStream_t stream) {
  if (batch_ == 0) return;
  // Append then attend, fused into one launch (same result as reshape_and_cache
  // followed by paged_decode_attention); with a shared prefix the cascaded entry,
  // which runs the plain one where the cascade would not pay.
  if (shared_blocks_ > 0) {
    ::paged_decode_attention_shared_prefix(
        out, q, key, value, static_cast<const int64_t*>(d_slots_), cache_.k_cache(layer),
        cache_.v_cache(layer), static_cast<const uint32_t*>(d_cu_), static_cast<const int32_t*>(d_table_),
        static_cast<int64_t>(max_blocks_), static_cast<int64_t>(cache_.num_blocks()),
        static_cast<int64_t>(batch_), static_cast<int64_t>(num_heads_),
        static_cast<int64_t>(cache_.num_kv_heads()), static_cast<int64_t>(cache_.head_dim()),
        static_cast<int64_t>(cache_.block_size()), static_cast<int64_t>(max_seqlen_k_), window_left,
        softmax_scale, static_cast<int64_t>(shared_blocks_), d_ws_, cap_ws_, cache_.dtype(), stream);
    check_lib("paged_decode_attention_shared_prefix");
    return;
  }
  ::paged_decode_attention_append(
      out, q, key, value, static_cast<const int64_t*>(d_slots_), cache_.k_cache(layer),
      cache_.v_cache(layer), static_cast<const uint32_t*>(d_cu_),
      static_cast<const int32_t*>(d_table_), static_cast<int64_t>(max_blocks_),
      static_cast<int64_t>(cache_.num_blocks()), static_cast<int64_t>(batch_),
      static_cast<int64_t>(num_heads_), static_cast<int64_t>(cache_.num_kv_heads()),
      static_cast<int64_t>(cache_.head_dim()), static_cast<int64_t>(cache_.block_size()),
      static_cast<int64_t>(max_seqlen_k_), window_left, softmax_scale, d_ws_, cap_ws_,
      cache_.dtype(), stream);
  check_lib("paged_decode_attention_append");
}

PrefillStep::PrefillStep(const PagedKVCache& cache, std::size_t num_heads)
    : cache_(cache), num_heads_(num_heads) {}

PrefillStep::~PrefillStep() {
  if (d_buf_) (void)hipFree(d_buf_);
}

void PrefillStep::upload(const AttnMetadata& meta, const std::vector<std::vector<int32_t>>& block_table,
                         const std::vector<int32_t>& positions, hipStream_t stream) {
  if (!meta.is_prefill) throw std::invalid_argument("PrefillStep needs prefill metadata");
  batch_ = meta.cu_seqlens_q.empty() ? 0 : meta.cu_seqlens_q.size() - 1;
  num_tokens_ = batch_ ? meta.cu_seqlens_q.back() : 0;
  if (batch_ == 0) return;
  if (block_table.size() != batch_ || positions.size() != num_tokens_ || meta.slot_mapping.size() != num_tokens_)
    throw std::invalid_argument("PrefillStep: block_table / positions / slot_mapping do not match the batch");
  const PaddedTable t = pad_block_table(block_table);
  max_blocks_ = t.width;
  max_seqlen_q_ = meta.max_seqlen_q;
  max_seqlen_k_ = meta.max_seqlen_k;
  // The previous step's asynchronous upload may still read the staging copies.
  check(hipStreamSynchronize(stream), "hipStreamSynchronize");
  h_cuq_ = meta.cu_seqlens_q;
  h_cuk_ = meta.cu_seqlens_k;
  h_table_ = t.data;
  h_pos_ = positions;
  h_slots_ = meta.slot_mapping;
  auto part = [](std::size_t bytes) { return round_up(std::max<std::size_t>(bytes, 1), 256); };
  off_cuk_ = part(h_cuq_.size() * 4);
  off_table_ = off_cuk_ + part(h_cuk_.size() * 4);
  off_pos_ = off_table_ + part(h_table_.size() * 4);
  off_slots_ = off_pos_ + part(h_pos_.size() * 4);
  const std::size_t total = off_slots_ + part(h_slots_.size() * 8);
  if (total > cap_) {
    if (d_buf_) check(hipFree(d_buf_), "hipFree");
    d_buf_ = nullptr;
    check(hipMalloc(&d_buf_, total), "hipMalloc(PrefillStep)");
    cap_ = total;
  }
  char* d = static_cast<char*>(d_buf_);
  check(hipMemcpyAsync(d, h_cuq_.data(), h_cuq_.size() * 4, hipMemcpyHostToDevice, stream), "upload cu_seqlens_q");
  check(hipMemcpyAsync(d + off_cuk_, h_cuk_.data(), h_cuk_.size() * 4, hipMemcpyHostToDevice, stream),
        "upload cu_seqlens_k");
  check(hipMemcpyAsync(d + off_table_, h_table_.data(), h_table_.size() * 4, hipMemcpyHostToDevice, stream),
        "upload block_table");
  check(hipMemcpyAsync(d + off_pos_, h_pos_.data(), h_pos_.size() * 4, hipMemcpyHostToDevice, stream),
        "upload positions");
  check(hipMemcpyAsync(d + off_slots_, h_slots_.data(), h_slots_.size() * 8, hipMemcpyHostToDevice, stream),
        "upload slot_mapping");
}

void PrefillStep::run_layer(std::size_t layer, const void* qkv, const void* q_norm_weight,
                            const void* k_norm_weight, double eps, const float* cos_sin,
                            std::size_t max_position, void* q_scratch, void* out, float softmax_scale,
                            int32_t window_left, hipStream_t stream) {
  if (batch_ == 0 || num_tokens_ == 0) return;
  const char* d = static_cast<const char*>(d_buf_);
  const int64_t Hq = static_cast<int64_t>(num_heads_), Hkv = static_cast<int64_t>(cache_.num_kv_heads()),
                D = static_cast<int64_t>(cache_.head_dim());
  ::qk_norm_rope_and_cache(q_scratch, nullptr, qkv, (Hq + 2 * Hkv) * D, q_norm_weight, k_norm_weight, eps,
                           cos_sin, static_cast<int64_t>(max_position),
                           reinterpret_cast<const int32_t*>(d + off_pos_), cache_.k_cache(layer),
                           cache_.v_cache(layer), reinterpret_cast<const int64_t*>(d + off_slots_),
                           static_cast<int64_t>(num_tokens_), Hq, Hkv, D, cache_.dtype(), stream);
  check_lib("qk_norm_rope_and_cache");
  ::paged_prefill_attention(out, q_scratch, cache_.k_cache(layer), cache_.v_cache(layer),
                            reinterpret_cast<const uint32_t*>(d), reinterpret_cast<const uint32_t*>(d + off_cuk_),
                            reinterpret_cast<const int32_t*>(d + off_table_), static_cast<int64_t>(max_blocks_),
                            static_cast<int64_t>(cache_.num_blocks()), static_cast<int64_t>(batch_), Hq, Hkv, D,
                            static_cast<int64_t>(cache_.block_size()), static_cast<int64_t>(max_seqlen_q_),
                            static_cast<int64_t>(max_seqlen_k_), window_left, softmax_scale, cache_.dtype(),
                            stream);
  check_lib("paged_prefill_attention");
}

}  // namespace oxide::host
