// Host side of the paged-KV path, in C++: the block pool with its chained
// prefix hash, slot mapping, attention metadata, block-table padding, and the
// physical cache buffer plus a decode-step driver over the C ABI.
//
// It mirrors the reference's host types (Rust there) so a C++ engine can drive
// the gfx950 kernels the way the reference's engine drives its CUDA ones:
//   BlockPool / Block          crates/vllm-oxide/src/engine/block_pool.rs:96-369
//   Sequence (block slicing)   crates/vllm-oxide/src/engine/sequence.rs:20,100-130
//   KvCacheManager             crates/vllm-oxide/src/engine/kv_cache_manager.rs:54-140
//   AttnMetadata + builders    crates/vllm-oxide/src/attention/metadata.rs:9-81
//   block_table_tensor padding crates/vllm-oxide/src/attention/flash_attn.rs:74-86
//   kv_cache_layout_shape      crates/vllm-oxide/src/utils.rs:46-61
//   PagedKVCache               crates/vllm-oxide/src/attention/mod.rs:48-112
//   RotaryEmbedding cache      crates/vllm-oxide/src/layers/rope.rs:50-83
// Fallible pool operations throw BlockPoolError where the reference returns
// Err(BlockPoolError); the messages name the same conditions.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <deque>
#include <optional>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

namespace oxide::host {

inline constexpr std::size_t kBlockSize = 256;  // sequence.rs:20

// [2, num_layers, num_blocks, block_size, num_kv_heads, head_dim] (dim 0: K, V).
std::array<std::size_t, 6> kv_cache_layout_shape(std::size_t num_layers, std::size_t num_blocks,
                                                 std::size_t block_size, std::size_t num_kv_heads,
                                                 std::size_t head_dim);
// Smallest multiple of m that is >= x (m > 0).
std::size_t round_up(std::size_t x, std::size_t m);

// XXH64 of `len` bytes (the 64-bit xxHash of the public specification).
uint64_t xxh64(const void* data, std::size_t len, uint64_t seed);

// RotaryEmbedding's cos_sin_cache (crates/vllm-oxide/src/layers/rope.rs:50-83):
// [max_position, rotary_dim] fp32, row t = [cos(t f_i) | sin(t f_i)] with
// f_i = 1 / base^(2i / rotary_dim), all in fp32.
std::vector<float> rope_cos_sin_cache(std::size_t max_position, std::size_t rotary_dim, float base);

// ------------------------------------------------------------------ metadata
struct AttnMetadata {
  bool is_prefill = false;
  std::vector<uint32_t> cu_seqlens_q;
  std::vector<uint32_t> cu_seqlens_k;
  std::size_t max_seqlen_q = 0;
  std::size_t max_seqlen_k = 0;
  std::vector<int64_t> slot_mapping;
  std::vector<std::vector<int32_t>> block_table;
};

AttnMetadata build_decode_metadata(const std::vector<uint32_t>& context_lens,
                                   const std::vector<std::vector<int32_t>>& block_table,
                                   const std::vector<int64_t>& slot_mapping);
AttnMetadata build_prefill_metadata(const std::vector<uint32_t>& scheduled_tokens,
                                    const std::vector<uint32_t>& kv_lengths,
                                    const std::vector<int64_t>& slot_mapping);

// Ragged rows padded with 0 to [rows, width] (row-major); throws on no rows,
// as the reference bails on an empty table.
struct PaddedTable {
  std::vector<int32_t> data;
  std::size_t rows = 0;
  std::size_t width = 0;
};
PaddedTable pad_block_table(const std::vector<std::vector<int32_t>>& block_table);

// ------------------------------------------------------------ block pool
struct Sequence {
  std::vector<uint32_t> token_ids;
  std::size_t num_tokens = 0;
  std::size_t num_cached_tokens = 0;
  std::size_t num_scheduled_tokens = 0;
  std::vector<std::size_t> block_table;

  explicit Sequence(std::vector<uint32_t> tokens = {});
  std::size_t num_blocks() const;               // ceil(num_tokens / 256)
  std::size_t last_block_num_tokens() const;
  std::vector<uint32_t> block(std::size_t i) const;  // tokens of logical block i
  void append_token(uint32_t token_id);
};

struct Block {
  std::size_t block_id = 0;
  std::size_t ref_count = 0;
  int64_t hash = -1;
  std::vector<uint32_t> token_ids;
};

class BlockPoolError : public std::runtime_error {
 public:
  explicit BlockPoolError(const std::string& m) : std::runtime_error("BlockPool: " + m) {}
};

class BlockPool {
 public:
  BlockPool(std::size_t num_blocks, std::size_t block_size);

  // XXH64 (seed 0) over prefix.to_le_bytes() (omitted when prefix == -1)
  // followed by each token's u32 little-endian bytes.
  static int64_t compute_hash(const std::vector<uint32_t>& token_ids, int64_t prefix);

  // Number of leading full blocks already cached, or nullopt if the pool
  // cannot hold the sequence.
  std::optional<std::size_t> can_allocate(const Sequence& seq) const;
  void allocate(Sequence& seq, std::size_t num_cached_blocks);
  void deallocate(Sequence& seq);
  bool can_append(const Sequence& seq) const;
  void may_append(Sequence& seq);  // new block iff num_tokens % block_size == 1
  void hash_blocks(Sequence& seq);

  // Copy-on-write sharing of whole block tables (parallel sampling, beam
  // search).  The reference's pool shares only full, hashed prefix blocks, so
  // it never writes into a shared block (its copy_blocks kernel has no
  // caller); these three calls add the missing write path.
  //   fork: `child` takes `parent`'s tokens and block table; every block gains
  //         a reference.
  //   can_append_cow / may_append_cow: call after appending a token to `seq`
  //         (num_tokens counts it).  A token that starts a block gets a fresh
  //         block (may_append); a token that lands in a block other tables
  //         still reference gets a private copy of it: the returned
  //         (src, dst) pair must be copied in the cache (copy_blocks) before the
  //         token's K/V are written.
  void fork(const Sequence& parent, Sequence& child);
  bool can_append_cow(const Sequence& seq) const;
  std::optional<std::pair<std::size_t, std::size_t>> may_append_cow(Sequence& seq);

  std::size_t num_free_blocks() const { return free_block_ids_.size(); }
  std::size_t num_blocks() const { return blocks_.size(); }
  std::size_t block_size() const { return block_size_; }
  const Block& block(std::size_t id) const { return blocks_.at(id); }
  bool is_used(std::size_t id) const { return used_block_ids_.count(id) != 0; }
  // Registers block `id` as holding `tokens` with chained hash `h` (what
  // hash_blocks does for one block).
  void register_hash(std::size_t id, int64_t h, std::vector<uint32_t> tokens);
  std::size_t allocate_block();  // pops the front of the free list

 private:
  void deallocate_block(std::size_t id);

  std::size_t block_size_;
  std::vector<Block> blocks_;
  std::unordered_map<int64_t, std::size_t> hash_to_block_id_;
  std::deque<std::size_t> free_block_ids_;
  std::unordered_set<std::size_t> used_block_ids_;
};

class KvCacheManager {
 public:
  KvCacheManager(std::size_t num_blocks, std::size_t block_size);
  std::optional<std::size_t> can_allocate(const Sequence& s) const { return pool_.can_allocate(s); }
  void allocate(Sequence& s, std::size_t cached) { pool_.allocate(s, cached); }
  void deallocate(Sequence& s) { pool_.deallocate(s); }
  bool can_append(const Sequence& s) const { return pool_.can_append(s); }
  void may_append(Sequence& s) { pool_.may_append(s); }
  void hash_blocks(Sequence& s) { pool_.hash_blocks(s); }
  void fork(const Sequence& parent, Sequence& child) { pool_.fork(parent, child); }
  bool can_append_cow(const Sequence& s) const { return pool_.can_append_cow(s); }
  std::optional<std::pair<std::size_t, std::size_t>> may_append_cow(Sequence& s) {
    return pool_.may_append_cow(s);
  }
  std::size_t num_free_blocks() const { return pool_.num_free_blocks(); }
  std::size_t block_size() const { return block_size_; }
  BlockPool& pool() { return pool_; }

  // slot[i] = block_table[(off+i)/bs]*bs + (off+i)%bs, or -1 past the table.
  std::vector<int64_t> compute_slot_mapping(const Sequence& seq, std::size_t token_offset,
                                            std::size_t num_tokens) const;

 private:
  BlockPool pool_;
  std::size_t block_size_;
};

}  // namespace oxide::host
