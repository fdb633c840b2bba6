// Block pool, sequence block slicing and slot mapping (host side).
// Semantics follow crates/vllm-oxide/src/engine/block_pool.rs:96-369,
// sequence.rs:100-130 and kv_cache_manager.rs:115-135.
#include <algorithm>
#include <cstring>

#include "oxide_host.hpp"

namespace oxide::host {

// ---------------------------------------------------------------- Sequence
Sequence::Sequence(std::vector<uint32_t> tokens)
    : token_ids(std::move(tokens)), num_tokens(token_ids.size()) {}

std::size_t Sequence::num_blocks() const { return (num_tokens + kBlockSize - 1) / kBlockSize; }

std::size_t Sequence::last_block_num_tokens() const {
  const std::size_t nb = num_blocks();
  return nb == 0 ? 0 : num_tokens - (nb - 1) * kBlockSize;
}

std::vector<uint32_t> Sequence::block(std::size_t i) const {
  const std::size_t start = i * kBlockSize;
  const std::size_t end = std::min(start + kBlockSize, num_tokens);
  return std::vector<uint32_t>(token_ids.begin() + start, token_ids.begin() + end);
}

void Sequence::append_token(uint32_t token_id) {
  token_ids.push_back(token_id);
  ++num_tokens;
}

// --------------------------------------------------------------- BlockPool
BlockPool::BlockPool(std::size_t num_blocks, std::size_t block_size) : block_size_(block_size) {
  blocks_.resize(num_blocks);
  for (std::size_t i = 0; i < num_blocks; ++i) {
    blocks_[i].block_id = i;
    free_block_ids_.push_back(i);
  }
}

int64_t BlockPool::compute_hash(const std::vector<uint32_t>& token_ids, int64_t prefix) {
  std::vector<uint8_t> bytes;
  bytes.reserve(8 + 4 * token_ids.size());
  if (prefix != -1) {
    const uint64_t p = static_cast<uint64_t>(prefix);
    for (int i = 0; i < 8; ++i) bytes.push_back(static_cast<uint8_t>(p >> (8 * i)));
  }
  for (uint32_t t : token_ids)
    for (int i = 0; i < 4; ++i) bytes.push_back(static_cast<uint8_t>(t >> (8 * i)));
  return static_cast<int64_t>(xxh64(bytes.data(), bytes.size(), 0));
}

std::size_t BlockPool::allocate_block() {
  if (free_block_ids_.empty()) throw BlockPoolError("no free blocks available");
  const std::size_t id = free_block_ids_.front();
  free_block_ids_.pop_front();
  Block& blk = blocks_[id];
  if (blk.hash != -1) {
    auto it = hash_to_block_id_.find(blk.hash);
    if (it != hash_to_block_id_.end() && it->second == id) hash_to_block_id_.erase(it);
  }
  blk.ref_count = 1;
  blk.hash = -1;
  blk.token_ids.clear();
  used_block_ids_.insert(id);
  return id;
}

void BlockPool::deallocate_block(std::size_t id) {
  if (used_block_ids_.erase(id) == 0)
    throw BlockPoolError("block " + std::to_string(id) + " is not in the used set (double-free?)");
  free_block_ids_.push_back(id);
}

std::optional<std::size_t> BlockPool::can_allocate(const Sequence& seq) const {
  const std::size_t nb = seq.num_blocks();
  if (nb == 0) return 0;
  int64_t h = -1;
  std::size_t cached = 0;
  std::size_t new_blocks = nb;
  for (std::size_t i = 0; i + 1 < nb; ++i) {  // the last (partial) block is never cached
    const std::vector<uint32_t> toks = seq.block(i);
    h = compute_hash(toks, h);
    auto it = hash_to_block_id_.find(h);
    if (it == hash_to_block_id_.end() || blocks_[it->second].token_ids != toks) break;
    ++cached;
    if (used_block_ids_.count(it->second)) --new_blocks;
  }
  if (free_block_ids_.size() < new_blocks) return std::nullopt;
  return cached;
}

void BlockPool::allocate(Sequence& seq, std::size_t num_cached_blocks) {
  if (!seq.block_table.empty()) throw BlockPoolError("sequence already has a block table");
  int64_t h = -1;
  for (std::size_t i = 0; i < num_cached_blocks; ++i) {
    h = compute_hash(seq.block(i), h);
    auto it = hash_to_block_id_.find(h);
    if (it == hash_to_block_id_.end()) throw BlockPoolError("cached block hash not found");
    const std::size_t id = it->second;
    if (used_block_ids_.count(id)) {
      ++blocks_[id].ref_count;
    } else {
      // Hashed earlier, since freed: move it from the free list to used.
      auto f = std::find(free_block_ids_.begin(), free_block_ids_.end(), id);
      if (f == free_block_ids_.end()) throw BlockPoolError("cached block not in free list");
      free_block_ids_.erase(f);
      blocks_[id].ref_count = 1;
      used_block_ids_.insert(id);
    }
    seq.block_table.push_back(id);
  }
  for (std::size_t i = num_cached_blocks; i < seq.num_blocks(); ++i)
    seq.block_table.push_back(allocate_block());
  seq.num_cached_tokens = num_cached_blocks * block_size_;
}

void BlockPool::deallocate(Sequence& seq) {
  for (auto it = seq.block_table.rbegin(); it != seq.block_table.rend(); ++it) {
    Block& blk = blocks_[*it];
    if (blk.ref_count == 0)
      throw BlockPoolError("block " + std::to_string(*it) + " already has ref_count 0 (double-free?)");
    if (--blk.ref_count == 0) deallocate_block(*it);
  }
  seq.num_cached_tokens = 0;
  seq.block_table.clear();
}

bool BlockPool::can_append(const Sequence& seq) const {
  const std::size_t need = seq.num_tokens % block_size_ == 1 ? 1 : 0;
  return free_block_ids_.size() >= need;
}

void BlockPool::may_append(Sequence& seq) {
  if (seq.num_tokens % block_size_ == 1) seq.block_table.push_back(allocate_block());
}

void BlockPool::fork(const Sequence& parent, Sequence& child) {
  if (!child.block_table.empty()) throw BlockPoolError("sequence already has a block table");
  for (std::size_t id : parent.block_table) {
    if (!used_block_ids_.count(id)) throw BlockPoolError("block " + std::to_string(id) + " is not in use");
    ++blocks_[id].ref_count;
  }
  child.token_ids = parent.token_ids;
  child.num_tokens = parent.num_tokens;
  child.num_cached_tokens = parent.num_cached_tokens;
  child.num_scheduled_tokens = 0;
  child.block_table = parent.block_table;
}

bool BlockPool::can_append_cow(const Sequence& seq) const {
  std::size_t need = 0;
  if (seq.num_tokens % block_size_ == 1) {
    need = 1;
  } else if (!seq.block_table.empty() && blocks_[seq.block_table.back()].ref_count > 1) {
    need = 1;
  }
  return free_block_ids_.size() >= need;
}

std::optional<std::pair<std::size_t, std::size_t>> BlockPool::may_append_cow(Sequence& seq) {
  if (seq.num_tokens % block_size_ == 1) {
    seq.block_table.push_back(allocate_block());
    return std::nullopt;
  }
  if (seq.block_table.empty()) return std::nullopt;
  const std::size_t src = seq.block_table.back();
  if (blocks_[src].ref_count <= 1) return std::nullopt;
  const std::size_t dst = allocate_block();
  --blocks_[src].ref_count;
  seq.block_table.back() = dst;
  return std::make_pair(src, dst);
}

void BlockPool::register_hash(std::size_t id, int64_t h, std::vector<uint32_t> tokens) {
  blocks_.at(id).hash = h;
  blocks_[id].token_ids = std::move(tokens);
  hash_to_block_id_[h] = id;
}

void BlockPool::hash_blocks(Sequence& seq) {
  const std::size_t start = seq.num_cached_tokens / block_size_;
  const std::size_t end = (seq.num_cached_tokens + seq.num_scheduled_tokens) / block_size_;
  if (start >= end) return;
  int64_t h = start > 0 ? blocks_[seq.block_table[start - 1]].hash : -1;
  for (std::size_t i = start; i < end; ++i) {
    std::vector<uint32_t> toks = seq.block(i);
    h = compute_hash(toks, h);
    register_hash(seq.block_table[i], h, std::move(toks));
  }
}

// ---------------------------------------------------------- KvCacheManager
KvCacheManager::KvCacheManager(std::size_t num_blocks, std::size_t block_size)
    : pool_(num_blocks, block_size), block_size_(block_size) {}

std::vector<int64_t> KvCacheManager::compute_slot_mapping(const Sequence& seq,
                                                          std::size_t token_offset,
                                                          std::size_t num_tokens) const {
  std::vector<int64_t> mapping;
  mapping.reserve(num_tokens);
  for (std::size_t i = 0; i < num_tokens; ++i) {
    const std::size_t abs_idx = token_offset + i;
    const std::size_t blk = abs_idx / block_size_;
    const std::size_t off = abs_idx % block_size_;
    mapping.push_back(blk < seq.block_table.size()
                          ? static_cast<int64_t>(seq.block_table[blk] * block_size_ + off)
                          : -1);
  }
  return mapping;
}

}  // namespace oxide::host
