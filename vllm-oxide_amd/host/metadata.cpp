// Attention metadata, block-table padding, layout helpers and XXH64 (host).
// Semantics follow crates/vllm-oxide/src/attention/metadata.rs:20-81,
// attention/flash_attn.rs:74-86 and utils.rs:27-61.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "oxide_host.hpp"
#include "oxide_paged_kv.h"

namespace oxide::host {

std::array<std::size_t, 6> kv_cache_layout_shape(std::size_t num_layers, std::size_t num_blocks,
                                                 std::size_t block_size, std::size_t num_kv_heads,
                                                 std::size_t head_dim) {
  return {2, num_layers, num_blocks, block_size, num_kv_heads, head_dim};
}

std::size_t round_up(std::size_t x, std::size_t m) { return (x + m - 1) / m * m; }

AttnMetadata build_decode_metadata(const std::vector<uint32_t>& context_lens,
                                   const std::vector<std::vector<int32_t>>& block_table,
                                   const std::vector<int64_t>& slot_mapping) {
  AttnMetadata m;
  m.is_prefill = false;
  m.cu_seqlens_q.assign(1, 0);
  m.cu_seqlens_k.assign(1, 0);
  for (uint32_t ctx : context_lens) {
    m.cu_seqlens_q.push_back(m.cu_seqlens_q.back() + 1);
    m.cu_seqlens_k.push_back(m.cu_seqlens_k.back() + ctx);
    if (ctx > m.max_seqlen_k) m.max_seqlen_k = ctx;
  }
  m.max_seqlen_q = 1;
  m.slot_mapping = slot_mapping;
  m.block_table = block_table;
  return m;
}

AttnMetadata build_prefill_metadata(const std::vector<uint32_t>& scheduled_tokens,
                                    const std::vector<uint32_t>& kv_lengths,
                                    const std::vector<int64_t>& slot_mapping) {
  AttnMetadata m;
  m.is_prefill = true;
  m.cu_seqlens_q.assign(1, 0);
  m.cu_seqlens_k.assign(1, 0);
  for (std::size_t i = 0; i < scheduled_tokens.size() && i < kv_lengths.size(); ++i) {
    m.cu_seqlens_q.push_back(m.cu_seqlens_q.back() + scheduled_tokens[i]);
    m.cu_seqlens_k.push_back(m.cu_seqlens_k.back() + kv_lengths[i]);
    if (scheduled_tokens[i] > m.max_seqlen_q) m.max_seqlen_q = scheduled_tokens[i];
    if (kv_lengths[i] > m.max_seqlen_k) m.max_seqlen_k = kv_lengths[i];
  }
  m.slot_mapping = slot_mapping;
  return m;
}

PaddedTable pad_block_table(const std::vector<std::vector<int32_t>>& block_table) {
  if (block_table.empty())
    throw std::invalid_argument("block_table must be non-empty for decode attention");
  PaddedTable t;
  t.rows = block_table.size();
  for (const auto& r : block_table) t.width = std::max(t.width, r.size());
  t.data.assign(t.rows * t.width, 0);
  // std::copy, not memcpy: an empty row's data() may be null.
  for (std::size_t b = 0; b < t.rows; ++b)
    std::copy(block_table[b].begin(), block_table[b].end(), t.data.begin() + b * t.width);
  return t;
}

// XXH64 from the public specification (64-bit variant): four 8-byte lanes over
// 32-byte stripes, merged, then the tail in 8-, 4- and 1-byte steps, then the
// avalanche.
namespace {
constexpr uint64_t kP1 = 0x9E3779B185EBCA87ULL, kP2 = 0xC2B2AE3D27D4EB4FULL,
                   kP3 = 0x165667B19E3779F9ULL, kP4 = 0x85EBCA77C2B2AE63ULL,
                   kP5 = 0x27D4EB2F165667C5ULL;
inline uint64_t rotl(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
inline uint64_t le64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
  return v;
}
inline uint32_t le32(const uint8_t* p) {
  return static_cast<uint32_t>(p[0]) | static_cast<uint32_t>(p[1]) << 8 |
         static_cast<uint32_t>(p[2]) << 16 | static_cast<uint32_t>(p[3]) << 24;
}
inline uint64_t lane_round(uint64_t acc, uint64_t in) { return rotl(acc + in * kP2, 31) * kP1; }
inline uint64_t merge_lane(uint64_t h, uint64_t v) { return (h ^ lane_round(0, v)) * kP1 + kP4; }
}  // namespace

uint64_t xxh64(const void* data, std::size_t len, uint64_t seed) {
  const uint8_t* p = static_cast<const uint8_t*>(data);
  const uint8_t* const end = p + len;
  uint64_t h;
  if (len >= 32) {
    uint64_t v[4] = {seed + kP1 + kP2, seed + kP2, seed, seed - kP1};
    for (; p + 32 <= end; p += 32)
      for (int i = 0; i < 4; ++i) v[i] = lane_round(v[i], le64(p + 8 * i));
    h = rotl(v[0], 1) + rotl(v[1], 7) + rotl(v[2], 12) + rotl(v[3], 18);
    for (int i = 0; i < 4; ++i) h = merge_lane(h, v[i]);
  } else {
    h = seed + kP5;
  }
  h += static_cast<uint64_t>(len);
  for (; p + 8 <= end; p += 8) h = rotl(h ^ lane_round(0, le64(p)), 27) * kP1 + kP4;
  if (p + 4 <= end) {
    h = rotl(h ^ (static_cast<uint64_t>(le32(p)) * kP1), 23) * kP2 + kP3;
    p += 4;
  }
  for (; p < end; ++p) h = rotl(h ^ (static_cast<uint64_t>(*p) * kP5), 11) * kP1;
  h ^= h >> 33;
  h *= kP2;
  h ^= h >> 29;
  h *= kP3;
  h ^= h >> 32;
  return h;
}

std::vector<float> rope_cos_sin_cache(std::size_t max_position, std::size_t rotary_dim, float base) {
  const std::size_t half = rotary_dim / 2;
  std::vector<float> cache(max_position * rotary_dim);
  for (std::size_t i = 0; i < half; ++i) {
    const float inv_freq = 1.0f / std::pow(base, static_cast<float>(2 * i) / static_cast<float>(rotary_dim));
    for (std::size_t t = 0; t < max_position; ++t) {
      const float f = static_cast<float>(t) * inv_freq;
      cache[t * rotary_dim + i] = std::cos(f);
      cache[t * rotary_dim + half + i] = std::sin(f);
    }
  }
  return cache;
}

}  // namespace oxide::host

extern "C" int oxide_rope_cos_sin_cache(float* cache, int64_t max_position, int64_t rotary_dim, float base) {
  if (!cache || max_position <= 0 || rotary_dim <= 0 || rotary_dim % 2 != 0) return OXIDE_ERR_INVALID_ARGUMENT;
  const std::vector<float> c = oxide::host::rope_cos_sin_cache(static_cast<std::size_t>(max_position),
                                                               static_cast<std::size_t>(rotary_dim), base);
  std::copy(c.begin(), c.end(), cache);
  return OXIDE_OK;
}
