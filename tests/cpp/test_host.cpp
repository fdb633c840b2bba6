// C++ tests of the host layer (vllm-oxide_amd/host), restating the reference's
// own unit tests.  `test_host cpu` runs the host-logic tests (no GPU calls);
// `test_host gpu` runs PagedKVCache / DecodeStep on device 0; `test_host hash
// <seed> <hex bytes>` prints one XXH64 digest (the pytest driver compares it
// with python-xxhash).
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include <atomic>
#include <thread>

#include "exact_div.hpp"
#include "oxide_host.hpp"
#include "paged_kv_cache.hpp"

using namespace oxide::host;

static int g_failures = 0;
#define CHECK(cond)                                                          \
  do {                                                                       \
    if (!(cond)) {                                                           \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);            \
      ++g_failures;                                                          \
    }                                                                        \
  } while (0)

template <class F>
static bool throws(F f) {
  try {
    f();
  } catch (const std::exception&) {
    return true;
  }
  return false;
}

static std::vector<uint32_t> iota(uint32_t a, uint32_t b) {
  std::vector<uint32_t> v;
  for (uint32_t i = a; i < b; ++i) v.push_back(i);
  return v;
}

// utils.rs:63-140
static void test_layout() {
  CHECK((kv_cache_layout_shape(28, 1024, 256, 4, 128) == std::array<std::size_t, 6>{2, 28, 1024, 256, 4, 128}));
  CHECK((kv_cache_layout_shape(1, 2, 3, 4, 5) == std::array<std::size_t, 6>{2, 1, 2, 3, 4, 5}));
  CHECK(round_up(0, 256) == 0 && round_up(256, 256) == 256 && round_up(1, 256) == 256);
  CHECK(round_up(255, 256) == 256 && round_up(257, 256) == 512 && round_up(41, 1) == 41);
  CHECK(round_up(4, 3) == 6 && round_up(7, 3) == 9 && round_up(3, 3) == 3);
}

// metadata.rs:82-218
static void test_metadata() {
  auto m = build_decode_metadata({5, 20, 3}, {{0}, {1, 2}, {3}}, {100, 200, 300});
  CHECK((m.cu_seqlens_q == std::vector<uint32_t>{0, 1, 2, 3}));
  CHECK((m.cu_seqlens_k == std::vector<uint32_t>{0, 5, 25, 28}));
  CHECK(m.max_seqlen_q == 1 && m.max_seqlen_k == 20 && !m.is_prefill);
  CHECK((m.slot_mapping == std::vector<int64_t>{100, 200, 300}));
  CHECK(m.block_table.size() == 3 && m.block_table[1].size() == 2);
  auto e = build_decode_metadata({}, {}, {});
  CHECK(e.cu_seqlens_q == std::vector<uint32_t>{0} && e.cu_seqlens_k == std::vector<uint32_t>{0});
  CHECK(e.max_seqlen_k == 0);
  auto p = build_prefill_metadata({4, 8, 3}, {4, 16, 3}, {0, 0, 0});
  CHECK((p.cu_seqlens_q == std::vector<uint32_t>{0, 4, 12, 15}));
  CHECK((p.cu_seqlens_k == std::vector<uint32_t>{0, 4, 20, 23}));
  CHECK(p.is_prefill && p.block_table.empty());
  auto q = build_prefill_metadata({4, 12, 3}, {4, 20, 3}, {});
  CHECK(q.max_seqlen_q == 12 && q.max_seqlen_k == 20);
  // flash_attn.rs:74-86: pad with 0; empty table is an error.
  auto t = pad_block_table({{7, 3}, {}, {1, 2, 9, 4}});
  CHECK(t.rows == 3 && t.width == 4);
  CHECK((t.data == std::vector<int32_t>{7, 3, 0, 0, 0, 0, 0, 0, 1, 2, 9, 4}));
  CHECK(throws([] { pad_block_table({}); }));
}

// kv_cache_manager.rs:254-322
static void test_slot_mapping() {
  KvCacheManager mgr(10, 256);
  Sequence s(iota(0, 10));
  s.block_table = {42};
  CHECK((mgr.compute_slot_mapping(s, 0, 3) == std::vector<int64_t>{42 * 256, 42 * 256 + 1, 42 * 256 + 2}));
  Sequence s2(iota(0, 300));
  s2.block_table = {10, 20};
  CHECK((mgr.compute_slot_mapping(s2, 254, 4) ==
         std::vector<int64_t>{10 * 256 + 254, 10 * 256 + 255, 20 * 256, 20 * 256 + 1}));
  Sequence s3(iota(0, 3 * 256 + 50));
  s3.block_table = {5, 6, 7, 8};
  auto full = mgr.compute_slot_mapping(s3, 0, 3 * 256 + 50);
  bool ok = full.size() == 3 * 256 + 50;
  for (std::size_t i = 0; ok && i < full.size(); ++i)
    ok = full[i] == static_cast<int64_t>(s3.block_table[i / 256] * 256 + i % 256);
  CHECK(ok);
  CHECK(mgr.compute_slot_mapping(Sequence({1, 2, 3}), 0, 0).empty());
  Sequence s4(iota(0, 10));
  s4.block_table = {1};
  CHECK(mgr.compute_slot_mapping(s4, 256, 1) == std::vector<int64_t>{-1});
}

// block_pool.rs:371-885
static void test_block_pool() {
  // compute_hash properties
  CHECK(BlockPool::compute_hash({1, 2, 3}, -1) != BlockPool::compute_hash({1, 2, 3}, 0));
  CHECK(BlockPool::compute_hash({1, 2, 3}, 0) != BlockPool::compute_hash({1, 2, 3}, 42));
  CHECK(BlockPool::compute_hash({10, 20, 30, 40}, 100) == BlockPool::compute_hash({10, 20, 30, 40}, 100));
  CHECK(BlockPool::compute_hash({1, 2, 3}, -1) != BlockPool::compute_hash({3, 2, 1}, -1));
  {  // prefix -1 omits the prefix bytes; prefix 0 prepends 8 zero bytes
    const uint8_t b78[8] = {7, 0, 0, 0, 8, 0, 0, 0};
    CHECK(BlockPool::compute_hash({7, 8}, -1) == static_cast<int64_t>(xxh64(b78, 8, 0)));
    uint8_t z[16] = {0};
    std::memcpy(z + 8, b78, 8);
    CHECK(BlockPool::compute_hash({7, 8}, 0) == static_cast<int64_t>(xxh64(z, 16, 0)));
  }
  {  // can_allocate
    BlockPool pool(10, 256);
    CHECK(pool.can_allocate(Sequence({})) == std::optional<std::size_t>(0));
    BlockPool small(2, 256);
    CHECK(!small.can_allocate(Sequence(iota(0, 4 * 256 + 1))).has_value());
    CHECK(small.can_allocate(Sequence(iota(0, 2 * 256))) == std::optional<std::size_t>(0));
  }
  {  // counts cached blocks
    BlockPool pool(10, 256);
    auto t1 = iota(0, 256), t2 = iota(256, 512);
    const int64_t h1 = BlockPool::compute_hash(t1, -1), h2 = BlockPool::compute_hash(t2, h1);
    const std::size_t b1 = pool.allocate_block(), b2 = pool.allocate_block();
    pool.register_hash(b1, h1, t1);
    pool.register_hash(b2, h2, t2);
    CHECK(pool.can_allocate(Sequence(iota(0, 3 * 256))) == std::optional<std::size_t>(2));
  }
  {  // allocate sets table and cached tokens; double allocate errors
    BlockPool pool(10, 256);
    Sequence s(iota(0, 3 * 256 + 50));
    CHECK(pool.can_allocate(s) == std::optional<std::size_t>(0));
    pool.allocate(s, 0);
    CHECK(s.block_table.size() == 4 && s.num_cached_tokens == 0);
    CHECK(throws([&] { pool.allocate(s, 0); }));
  }
  {  // shared prefix: ref counts, release only at zero
    BlockPool pool(10, 256);
    auto prefix = iota(0, 256);
    const int64_t h = BlockPool::compute_hash(prefix, -1);
    Sequence a(prefix);
    pool.allocate(a, 0);
    const std::size_t id = a.block_table[0];
    pool.register_hash(id, h, prefix);
    auto tb = prefix;
    tb.push_back(999);
    Sequence b(tb);
    const auto nc = pool.can_allocate(b);
    CHECK(nc == std::optional<std::size_t>(1));
    pool.allocate(b, *nc);
    CHECK(pool.block(id).ref_count == 2 && b.block_table[0] == id && b.block_table[1] != id);
    CHECK(b.num_cached_tokens == 256);
    pool.deallocate(a);
    CHECK(pool.block(id).ref_count == 1 && pool.is_used(id));
    pool.deallocate(b);
    CHECK(pool.block(id).ref_count == 0 && !pool.is_used(id));
    CHECK(pool.block(id).token_ids == prefix);  // the original block's tokens are untouched
    // The freed, still-hashed block is found again and moved back from the free list.
    Sequence c(tb);
    CHECK(pool.can_allocate(c) == std::optional<std::size_t>(1));
    pool.allocate(c, 1);
    CHECK(c.block_table[0] == id && pool.block(id).ref_count == 1);
  }
  {  // deallocate releases; twice is a no-op
    BlockPool pool(5, 256);
    Sequence s(iota(0, 2 * 256 + 1));
    pool.allocate(s, 0);
    CHECK(pool.num_free_blocks() == 2);
    pool.deallocate(s);
    CHECK(pool.num_free_blocks() == 5 && s.block_table.empty() && s.num_cached_tokens == 0);
    pool.deallocate(s);
    CHECK(s.block_table.empty());
  }
  {  // can_append / may_append: a new block iff num_tokens % 256 == 1
    BlockPool pool(1, 256);
    Sequence s(iota(0, 256));
    pool.allocate(s, 0);
    CHECK(pool.num_free_blocks() == 0 && pool.can_append(s));
    s.append_token(7);  // 257 tokens: the next token opens block 1
    CHECK(!pool.can_append(s));
    CHECK(throws([&] { pool.may_append(s); }));
    BlockPool pool2(2, 256);
    Sequence t(iota(0, 256));
    pool2.allocate(t, 0);
    t.append_token(7);
    pool2.may_append(t);
    CHECK(t.block_table.size() == 2 && pool2.num_free_blocks() == 0);
    t.append_token(8);  // 258: no new block
    pool2.may_append(t);
    CHECK(t.block_table.size() == 2);
  }
  {  // hash_blocks: incremental chain equals one pass
    BlockPool p1(10, 256), p2(10, 256);
    Sequence a(iota(0, 3 * 256)), b(iota(0, 3 * 256));
    p1.allocate(a, 0);
    p2.allocate(b, 0);
    a.num_cached_tokens = 0;
    a.num_scheduled_tokens = 3 * 256;
    p1.hash_blocks(a);
    b.num_cached_tokens = 0;
    b.num_scheduled_tokens = 256;
    p2.hash_blocks(b);
    b.num_cached_tokens = 256;
    b.num_scheduled_tokens = 2 * 256;
    p2.hash_blocks(b);
    for (int i = 0; i < 3; ++i) {
      CHECK(p1.block(a.block_table[i]).hash != -1);
      CHECK(p1.block(a.block_table[i]).hash == p2.block(b.block_table[i]).hash);
    }
    int64_t h = -1;
    for (int i = 0; i < 3; ++i) h = BlockPool::compute_hash(a.block(i), h);
    CHECK(p1.block(a.block_table[2]).hash == h);
  }
  {  // FIFO free list: freed blocks go to the back
    BlockPool pool(3, 256);
    const std::size_t x = pool.allocate_block();
    CHECK(x == 0);
    Sequence s(iota(0, 10));
    s.block_table = {x};
    pool.deallocate(s);
    CHECK(pool.allocate_block() == 1 && pool.allocate_block() == 2 && pool.allocate_block() == 0);
  }
}

// ------------------------------------------------------------------- GPU
// Copy-on-write sharing: fork, then appends into shared and private blocks.
static void test_cow() {
  BlockPool pool(8, 256);
  Sequence parent(iota(0, 300));
  pool.allocate(parent, 0);  // blocks 0, 1
  CHECK(parent.block_table.size() == 2 && pool.num_free_blocks() == 6);
  Sequence child;
  pool.fork(parent, child);
  CHECK(child.block_table == parent.block_table && child.num_tokens == 300);
  CHECK(pool.block(parent.block_table[0]).ref_count == 2 && pool.block(parent.block_table[1]).ref_count == 2);
  CHECK(pool.num_free_blocks() == 6);
  CHECK(throws([&] { pool.fork(parent, child); }));  // child already has a table
  // Parent appends token 300 into the shared partial block 1: private copy.
  const std::size_t shared = parent.block_table[1];
  parent.append_token(1000);
  CHECK(pool.can_append_cow(parent));
  const auto cp = pool.may_append_cow(parent);
  CHECK(cp.has_value() && cp->first == shared && cp->second != shared);
  CHECK(parent.block_table[1] == cp->second && child.block_table[1] == shared);
  CHECK(pool.block(shared).ref_count == 1 && pool.block(cp->second).ref_count == 1);
  CHECK(pool.num_free_blocks() == 5);
  // Child's block is now private: no copy.  Block 0 stays shared (full, never written).
  child.append_token(2000);
  CHECK(!pool.may_append_cow(child).has_value());
  CHECK(pool.block(parent.block_table[0]).ref_count == 2);
  // A token that starts a block gets a fresh one, no copy.
  Sequence s2(iota(0, 256));
  pool.allocate(s2, 0);
  s2.append_token(7);
  CHECK(s2.num_tokens % 256 == 1);
  CHECK(!pool.may_append_cow(s2).has_value() && s2.block_table.size() == 2);
  // No free block: can_append_cow refuses a copy.
  BlockPool tiny(1, 256);
  Sequence a(iota(0, 10));
  tiny.allocate(a, 0);
  Sequence b;
  tiny.fork(a, b);
  b.append_token(1);
  CHECK(!tiny.can_append_cow(b));
  CHECK(throws([&] { tiny.may_append_cow(b); }));
  // Release everything: every block returns to the free list exactly once.
  pool.deallocate(parent);
  pool.deallocate(child);
  pool.deallocate(s2);
  CHECK(pool.num_free_blocks() == 8);
}

// Randomised sequences of allocate / fork / append (with CoW) / deallocate:
// after every operation each block's ref_count equals the number of live block
// tables holding it, used blocks are exactly those with references, and the
// free list holds the rest; at the end everything is free again.
static void test_pool_random_ops() {
  const std::size_t NB = 24;
  BlockPool pool(NB, kBlockSize);  // Sequence counts blocks of kBlockSize (sequence.rs:20)
  std::vector<Sequence> live;
  std::size_t copies = 0, new_blocks = 0;
  uint64_t s = 99;
  auto rnd = [&s](uint64_t n) {
    s = s * 6364136223846793005ULL + 1442695040888963407ULL;
    return static_cast<std::size_t>((s >> 33) % n);
  };
  auto check_invariants = [&]() {
    std::vector<std::size_t> refs(NB, 0);
    for (const auto& q : live)
      for (std::size_t id : q.block_table) ++refs[id];
    std::size_t used = 0;
    for (std::size_t id = 0; id < NB; ++id) {
      CHECK(pool.block(id).ref_count == refs[id]);
      CHECK(pool.is_used(id) == (refs[id] > 0));
      used += refs[id] > 0;
    }
    CHECK(pool.num_free_blocks() + used == NB);
  };
  for (int step = 0; step < 20000; ++step) {
    const std::size_t op = rnd(10);
    if (op < 3) {  // new sequence
      // Half of them end at or next to a block boundary, so appends cross it.
      const std::size_t n = rnd(2) ? 1 + rnd(700) : kBlockSize * (1 + rnd(2)) - rnd(2);
      Sequence q(iota(0, static_cast<uint32_t>(n)));
      const auto cached = pool.can_allocate(q);
      if (cached) {
        pool.allocate(q, *cached);
        live.push_back(q);
      }
    } else if (op < 5 && !live.empty()) {  // fork
      Sequence child;
      pool.fork(live[rnd(live.size())], child);
      live.push_back(child);
    } else if (op < 8 && !live.empty()) {  // append tokens, one at a time
      Sequence& q = live[rnd(live.size())];
      q.append_token(static_cast<uint32_t>(rnd(1000)));
      if (pool.can_append_cow(q)) {
        const std::size_t before = q.block_table.size();
        if (pool.may_append_cow(q)) ++copies;
        if (q.block_table.size() > before) ++new_blocks;
        CHECK(q.block_table.size() == q.num_blocks());
      } else {
        q.token_ids.pop_back();  // no room: undo (the scheduler would preempt)
        --q.num_tokens;
      }
    } else if (!live.empty()) {  // finish a sequence
      const std::size_t i = rnd(live.size());
      pool.deallocate(live[i]);
      live.erase(live.begin() + static_cast<std::ptrdiff_t>(i));
    }
    check_invariants();
  }
  for (auto& q : live) pool.deallocate(q);
  live.clear();
  check_invariants();
  CHECK(pool.num_free_blocks() == NB);
  std::printf("random ops: %zu copies, %zu new blocks\n", copies, new_blocks);
  CHECK(copies > 20 && new_blocks > 10);  // both append paths were exercised
}

static uint16_t f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
static float bf2f(uint16_t h) {
  const uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// attention/mod.rs:161-230 reshape_and_cache_writes_correct_slots, through PagedKVCache.
static void test_gpu_append_known_answer() {
  const std::size_t H = 2, D = 64, T = 3;
  PagedKVCache cache(1, 4, 256, H, D, OXIDE_DTYPE_BF16);
  CHECK((cache.buffer_shape() == std::array<std::size_t, 6>{2, 1, 4, 256, 2, 64}));
  std::vector<uint16_t> key(T * H * D), val(T * H * D);
  for (std::size_t i = 0; i < key.size(); ++i) {
    key[i] = f2bf(static_cast<float>(i));
    val[i] = f2bf(1000.f + static_cast<float>(i));
  }
  const std::vector<int64_t> slots = {0, 256, 512};
  void *dk, *dv, *ds;
  (void)hipMalloc(&dk, key.size() * 2);
  (void)hipMalloc(&dv, val.size() * 2);
  (void)hipMalloc(&ds, 3 * 8);
  (void)hipMemcpy(dk, key.data(), key.size() * 2, hipMemcpyHostToDevice);
  (void)hipMemcpy(dv, val.data(), val.size() * 2, hipMemcpyHostToDevice);
  (void)hipMemcpy(ds, slots.data(), 3 * 8, hipMemcpyHostToDevice);
  cache.reshape_and_cache(0, dk, dv, static_cast<const int64_t*>(ds), T, nullptr);
  const std::size_t view = 4 * 256 * H * D;
  std::vector<uint16_t> kc(view), vc(view);
  (void)hipMemcpy(kc.data(), cache.k_cache(0), view * 2, hipMemcpyDeviceToHost);
  (void)hipMemcpy(vc.data(), cache.v_cache(0), view * 2, hipMemcpyDeviceToHost);
  const std::size_t row = H * D;
  // k[0,0] == key[0], k[1,0] == key[1], v[2,0] == value[2], max diff 0.
  CHECK(std::memcmp(kc.data() + 0 * 256 * row, key.data() + 0 * row, row * 2) == 0);
  CHECK(std::memcmp(kc.data() + 1 * 256 * row, key.data() + 1 * row, row * 2) == 0);
  CHECK(std::memcmp(vc.data() + 2 * 256 * row, val.data() + 2 * row, row * 2) == 0);
  std::size_t nonzero = 0;
  for (uint16_t x : kc) nonzero += x != 0;
  std::size_t want = 0;
  for (uint16_t x : key) want += x != 0;
  CHECK(nonzero == want);
  (void)hipFree(dk);
  (void)hipFree(dv);
  (void)hipFree(ds);
}

// attention/mod.rs:277-323 flash_attn_decode_runs (ctx 32, 4 heads, 4 kv heads,
// D 64): through DecodeStep, checked against an in-test fp64 softmax.
// Copy-on-write copies in every layer with one launch (copy_blocks_all_layers).
static void test_gpu_cow_all_layers() {
  const std::size_t L = 3, NB = 4, BS = 16, H = 2, D = 64;
  PagedKVCache cache(L, NB, BS, H, D, OXIDE_DTYPE_BF16);
  const std::size_t blk = BS * H * D, half = L * NB * blk;
  std::vector<uint16_t> host(2 * half);
  for (std::size_t i = 0; i < host.size(); ++i) host[i] = static_cast<uint16_t>(i * 2654435761u >> 16);
  void* base = cache.k_cache(0);
  (void)hipMemcpy(base, host.data(), host.size() * 2, hipMemcpyHostToDevice);
  cache.copy_blocks_all_layers({{1, 2}, {3, 0}}, nullptr);
  (void)hipDeviceSynchronize();
  std::vector<uint16_t> got(host.size());
  (void)hipMemcpy(got.data(), base, got.size() * 2, hipMemcpyDeviceToHost);
  std::vector<uint16_t> want = host;
  for (std::size_t kv = 0; kv < 2; ++kv)
    for (std::size_t l = 0; l < L; ++l) {
      const std::size_t off = kv * half + l * NB * blk;
      std::memcpy(&want[off + 2 * blk], &host[off + 1 * blk], blk * 2);
      std::memcpy(&want[off + 0 * blk], &host[off + 3 * blk], blk * 2);
    }
  CHECK(got == want);
  CHECK(throws([&] { cache.copy_blocks_all_layers({{1, 4}}, nullptr); }));
  CHECK(throws([&] { cache.copy_blocks_all_layers({{1, 2}, {2, 3}}, nullptr); }));  // dst 2 is a src
  CHECK(throws([&] { cache.copy_blocks_all_layers({{1, 2}, {3, 2}}, nullptr); }));  // dst 2 twice
}

static void test_gpu_decode_step() {
  const std::size_t Hq = 4, H = 4, D = 64, ctx = 32;
  PagedKVCache cache(2, 1, 256, H, D, OXIDE_DTYPE_BF16);
  DecodeStep step(cache, Hq);
  // Fill keys 0..30 through appends of a 31-token "prefill", then decode token 31.
  uint64_t s = 12345;
  auto rnd = [&s]() {
    s = s * 6364136223846793005ULL + 1442695040888963407ULL;
    return static_cast<float>(static_cast<int64_t>(s >> 11) % 2000 - 1000) / 1000.f;
  };
  std::vector<uint16_t> k(ctx * H * D), v(ctx * H * D), q(Hq * D);
  for (auto& x : k) x = f2bf(rnd());
  for (auto& x : v) x = f2bf(rnd());
  for (auto& x : q) x = f2bf(rnd());
  std::vector<int64_t> prefill_slots;
  for (std::size_t i = 0; i + 1 < ctx; ++i) prefill_slots.push_back(static_cast<int64_t>(i));
  void *dk, *dv, *dq, *dout, *ds;
  (void)hipMalloc(&dk, k.size() * 2);
  (void)hipMalloc(&dv, v.size() * 2);
  (void)hipMalloc(&dq, q.size() * 2);
  (void)hipMalloc(&dout, q.size() * 2);
  (void)hipMalloc(&ds, prefill_slots.size() * 8);
  (void)hipMemcpy(dk, k.data(), k.size() * 2, hipMemcpyHostToDevice);
  (void)hipMemcpy(dv, v.data(), v.size() * 2, hipMemcpyHostToDevice);
  (void)hipMemcpy(dq, q.data(), q.size() * 2, hipMemcpyHostToDevice);
  (void)hipMemcpy(ds, prefill_slots.data(), prefill_slots.size() * 8, hipMemcpyHostToDevice);
  for (std::size_t layer = 0; layer < 2; ++layer)
    cache.reshape_and_cache(layer, dk, dv, static_cast<const int64_t*>(ds), ctx - 1, nullptr);
  // Decode step: the new token (row 31 of k/v) goes to slot 31, then attention over 32 keys.
  KvCacheManager mgr(1, 256);
  Sequence seq(iota(0, ctx));
  seq.block_table = {0};
  const auto slot = mgr.compute_slot_mapping(seq, ctx - 1, 1);
  CHECK(slot == std::vector<int64_t>{31});
  step.upload(build_decode_metadata({static_cast<uint32_t>(ctx)}, {{0}}, slot), nullptr);
  const float scale = 1.f / std::sqrt(static_cast<float>(D));
  const char* knew = static_cast<const char*>(dk) + (ctx - 1) * H * D * 2;
  const char* vnew = static_cast<const char*>(dv) + (ctx - 1) * H * D * 2;
  for (std::size_t layer = 0; layer < 2; ++layer) {
    step.run_layer(layer, dq, knew, vnew, dout, scale, -1, nullptr);
    std::vector<uint16_t> out(q.size());
    (void)hipMemcpy(out.data(), dout, out.size() * 2, hipMemcpyDeviceToHost);
    double max_err = 0;
    for (std::size_t h = 0; h < Hq; ++h) {
      const std::size_t kh = h / (Hq / H);
      std::vector<double> sc(ctx);
      double mx = -1e300;
      for (std::size_t j = 0; j < ctx; ++j) {
        double dot = 0;
        for (std::size_t d = 0; d < D; ++d)
          dot += static_cast<double>(bf2f(q[h * D + d])) * bf2f(k[(j * H + kh) * D + d]);
        sc[j] = dot * scale;
        mx = std::max(mx, sc[j]);
      }
      double l = 0;
      for (auto& x : sc) l += (x = std::exp(x - mx));
      for (std::size_t d = 0; d < D; ++d) {
        double o = 0;
        for (std::size_t j = 0; j < ctx; ++j) o += sc[j] / l * bf2f(v[(j * H + kh) * D + d]);
        const double got = bf2f(out[h * D + d]);
        CHECK(!std::isnan(got));
        max_err = std::max(max_err, std::fabs(got - o));
      }
    }
    CHECK(max_err <= 2e-2);
  }
  for (void* p : {dk, dv, dq, dout, ds}) (void)hipFree(p);
}

// DecodeStep over a batch whose block tables share their first 16 blocks (one
// cached 4096-token prompt, block_pool.rs:133-142 sharing; each sequence's own
// blocks after it): upload counts the shared blocks, run_layer takes the cascaded
// entry (the plan runs the cascade at this size), and the output matches the plain
// entry's on the same cache within the attention tolerance.
static void test_gpu_decode_step_shared_prefix() {
  const std::size_t Hq = 32, H = 8, D = 128, BS = 256, B = 64, S = 16;
  std::vector<uint32_t> lens(B);
  std::vector<std::vector<int32_t>> tables(B);
  int32_t next = static_cast<int32_t>(S);
  for (std::size_t b = 0; b < B; ++b) {
    lens[b] = static_cast<uint32_t>(S * BS + 1 + (b * 37) % 900);
    for (std::size_t j = 0; j < S; ++j) tables[b].push_back(static_cast<int32_t>(j));
    for (std::size_t j = S * BS; j < lens[b]; j += BS) tables[b].push_back(next++);
  }
  const std::size_t NB = static_cast<std::size_t>(next);
  PagedKVCache cache(1, NB, BS, H, D, OXIDE_DTYPE_BF16);
  DecodeStep step(cache, Hq);
  uint64_t s = 99;
  auto rnd = [&s]() {
    s = s * 6364136223846793005ULL + 1442695040888963407ULL;
    return static_cast<float>(static_cast<int64_t>(s >> 11) % 2000 - 1000) / 1000.f;
  };
  const std::size_t cache_elems = NB * BS * H * D;
  std::vector<uint16_t> host(cache_elems);
  for (void* dst : {cache.k_cache(0), cache.v_cache(0)}) {
    for (auto& x : host) x = f2bf(rnd());
    (void)hipMemcpy(dst, host.data(), host.size() * 2, hipMemcpyHostToDevice);
  }
  std::vector<uint16_t> q(B * Hq * D), kn(B * H * D), vn(B * H * D);
  for (auto& x : q) x = f2bf(rnd());
  for (auto& x : kn) x = f2bf(rnd());
  for (auto& x : vn) x = f2bf(rnd());
  std::vector<int64_t> slots(B);
  for (std::size_t b = 0; b < B; ++b)
    slots[b] = static_cast<int64_t>(tables[b][(lens[b] - 1) / BS]) * BS + (lens[b] - 1) % BS;
  void *dq, *dk, *dv, *do1, *do2;
  (void)hipMalloc(&dq, q.size() * 2);
  (void)hipMalloc(&dk, kn.size() * 2);
  (void)hipMalloc(&dv, vn.size() * 2);
  (void)hipMalloc(&do1, q.size() * 2);
  (void)hipMalloc(&do2, q.size() * 2);
  (void)hipMemcpy(dq, q.data(), q.size() * 2, hipMemcpyHostToDevice);
  (void)hipMemcpy(dk, kn.data(), kn.size() * 2, hipMemcpyHostToDevice);
  (void)hipMemcpy(dv, vn.data(), vn.size() * 2, hipMemcpyHostToDevice);
  const AttnMetadata meta = build_decode_metadata(lens, tables, slots);
  step.upload(meta, nullptr);
  CHECK(step.shared_blocks() == S);
  const float scale = 1.f / std::sqrt(static_cast<float>(D));
  CHECK(paged_decode_attention_shared_prefix_plan(B, Hq, H, D, BS, meta.max_seqlen_k, S) != 3);
  step.run_layer(0, dq, dk, dv, do1, scale, -1, nullptr);
  CHECK(hipDeviceSynchronize() == hipSuccess);
  // The plain entry on the same cache (the new tokens are in place now).
  const PaddedTable t = pad_block_table(tables);
  void *dcu, *dtab, *dws;
  const std::size_t ws = paged_decode_attention_workspace_size(B, Hq, H, D, meta.max_seqlen_k);
  (void)hipMalloc(&dcu, meta.cu_seqlens_k.size() * 4);
  (void)hipMalloc(&dtab, t.data.size() * 4);
  (void)hipMalloc(&dws, ws);
  (void)hipMemcpy(dcu, meta.cu_seqlens_k.data(), meta.cu_seqlens_k.size() * 4, hipMemcpyHostToDevice);
  (void)hipMemcpy(dtab, t.data.data(), t.data.size() * 4, hipMemcpyHostToDevice);
  paged_decode_attention(do2, dq, cache.k_cache(0), cache.v_cache(0), static_cast<const uint32_t*>(dcu),
                         static_cast<const int32_t*>(dtab), static_cast<int64_t>(t.width), static_cast<int64_t>(NB),
                         B, Hq, H, D, BS, meta.max_seqlen_k, -1, scale, dws, ws, OXIDE_DTYPE_BF16, nullptr);
  CHECK(oxide_last_error() == OXIDE_OK);
  CHECK(hipDeviceSynchronize() == hipSuccess);
  std::vector<uint16_t> o1(q.size()), o2(q.size());
  (void)hipMemcpy(o1.data(), do1, o1.size() * 2, hipMemcpyDeviceToHost);
  (void)hipMemcpy(o2.data(), do2, o2.size() * 2, hipMemcpyDeviceToHost);
  double max_err = 0;
  for (std::size_t i = 0; i < o1.size(); ++i) {
    CHECK(!std::isnan(bf2f(o1[i])));
    max_err = std::max(max_err, static_cast<double>(std::fabs(bf2f(o1[i]) - bf2f(o2[i]))));
  }
  CHECK(max_err <= 2e-2);
  std::printf("decode step, shared prefix: %zu shared blocks, max |cascade - plain| %.3g\n", step.shared_blocks(),
              max_err);
  for (void* p : {dq, dk, dv, do1, do2, dcu, dtab, dws}) (void)hipFree(p);
}

// PrefillStep: a 24-token prompt behind a 40-token cached prefix (two sequences'
// worth of checks in one: the prefix keys come from the cache, the prompt's from
// the append).  Positions 0 and no q/k norm make the prologue an exact split of
// the qkv rows, so the output is checked against an in-test fp64 causal softmax.
static void test_gpu_prefill_step() {
  const std::size_t Hq = 4, H = 2, D = 64, BS = 16, P = 40, T = 24, L = P + T;
  PagedKVCache cache(1, 8, BS, H, D, OXIDE_DTYPE_BF16);
  uint64_t s = 777;
  auto rnd = [&s]() {
    s = s * 6364136223846793005ULL + 1442695040888963407ULL;
    return static_cast<float>(static_cast<int64_t>(s >> 11) % 2000 - 1000) / 1000.f;
  };
  // Logical block i of the sequence -> physical block table[i].
  const std::vector<int32_t> table = {5, 2, 7, 0};
  auto slot_of = [&](std::size_t j) { return static_cast<int64_t>(table[j / BS]) * BS + j % BS; };
  std::vector<uint16_t> kall(L * H * D), vall(L * H * D), qkv(T * (Hq + 2 * H) * D), q(T * Hq * D);
  for (auto& x : kall) x = f2bf(rnd());
  for (auto& x : vall) x = f2bf(rnd());
  for (std::size_t t = 0; t < T; ++t) {
    uint16_t* row = qkv.data() + t * (Hq + 2 * H) * D;
    for (std::size_t i = 0; i < Hq * D; ++i) q[t * Hq * D + i] = row[i] = f2bf(rnd());
    std::memcpy(row + Hq * D, kall.data() + (P + t) * H * D, H * D * 2);
    std::memcpy(row + (Hq + H) * D, vall.data() + (P + t) * H * D, H * D * 2);
  }
  // The prefix is already in the cache.
  std::vector<int64_t> pslots;
  for (std::size_t j = 0; j < P; ++j) pslots.push_back(slot_of(j));
  void *dk, *dv, *ds, *dqkv, *dq, *dout, *dcs;
  (void)hipMalloc(&dk, P * H * D * 2);
  (void)hipMalloc(&dv, P * H * D * 2);
  (void)hipMalloc(&ds, P * 8);
  (void)hipMemcpy(dk, kall.data(), P * H * D * 2, hipMemcpyHostToDevice);
  (void)hipMemcpy(dv, vall.data(), P * H * D * 2, hipMemcpyHostToDevice);
  (void)hipMemcpy(ds, pslots.data(), P * 8, hipMemcpyHostToDevice);
  cache.reshape_and_cache(0, dk, dv, static_cast<const int64_t*>(ds), P, nullptr);
  (void)hipMalloc(&dqkv, qkv.size() * 2);
  (void)hipMalloc(&dq, T * Hq * D * 2);
  (void)hipMalloc(&dout, T * Hq * D * 2);
  (void)hipMemcpy(dqkv, qkv.data(), qkv.size() * 2, hipMemcpyHostToDevice);
  const std::vector<float> cs = rope_cos_sin_cache(8, D, 1e6f);
  (void)hipMalloc(&dcs, cs.size() * 4);
  (void)hipMemcpy(dcs, cs.data(), cs.size() * 4, hipMemcpyHostToDevice);
  std::vector<int64_t> slots;
  for (std::size_t t = 0; t < T; ++t) slots.push_back(slot_of(P + t));
  PrefillStep step(cache, Hq);
  step.upload(build_prefill_metadata({static_cast<uint32_t>(T)}, {static_cast<uint32_t>(L)}, slots), {table},
              std::vector<int32_t>(T, 0), nullptr);
  const float scale = 1.f / std::sqrt(static_cast<float>(D));
  step.run_layer(0, dqkv, nullptr, nullptr, 1e-6, static_cast<const float*>(dcs), 8, dq, dout, scale, -1, nullptr);
  std::vector<uint16_t> out(T * Hq * D);
  (void)hipMemcpy(out.data(), dout, out.size() * 2, hipMemcpyDeviceToHost);
  double max_err = 0;
  for (std::size_t t = 0; t < T; ++t)
    for (std::size_t h = 0; h < Hq; ++h) {
      const std::size_t kh = h / (Hq / H), nk = P + t + 1;  // causal, aligned bottom-right
      std::vector<double> sc(nk);
      double mx = -1e300, l = 0;
      for (std::size_t j = 0; j < nk; ++j) {
        double dot = 0;
        for (std::size_t d = 0; d < D; ++d)
          dot += static_cast<double>(bf2f(q[(t * Hq + h) * D + d])) * bf2f(kall[(j * H + kh) * D + d]);
        mx = std::max(mx, sc[j] = dot * scale);
      }
      for (auto& x : sc) l += (x = std::exp(x - mx));
      for (std::size_t d = 0; d < D; ++d) {
        double o = 0;
        for (std::size_t j = 0; j < nk; ++j) o += sc[j] / l * bf2f(vall[(j * H + kh) * D + d]);
        max_err = std::max(max_err, std::fabs(bf2f(out[(t * Hq + h) * D + d]) - o));
      }
    }
  CHECK(max_err <= 2e-2);
  // The prompt's K/V landed in their slots.
  std::vector<uint16_t> kc(8 * BS * H * D);
  (void)hipMemcpy(kc.data(), cache.k_cache(0), kc.size() * 2, hipMemcpyDeviceToHost);
  CHECK(std::memcmp(kc.data() + slot_of(L - 1) * H * D, kall.data() + (L - 1) * H * D, H * D * 2) == 0);
  for (void* ptr : {dk, dv, ds, dqkv, dq, dout, dcs}) (void)hipFree(ptr);
}

// The fast divide of the attention prologue (exact_div.hpp) against the
// correctly rounded x / b.  The quotient's significand depends only on the
// significands of x and b while every step stays normal, so checking every
// f16 significand of x (a superset of bf16's) against every fp32 significand
// of b ("div full", 8.6e9 pairs) covers the whole domain; the default run
// takes every 97th b significand.  Edge exponents and signed zeros on top.
static float u2f(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
static void test_exact_div(bool full) {
  const uint32_t step = full ? 1 : 97;
  std::atomic<long long> bad{0}, checked{0};
  const unsigned nth = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
  std::vector<std::thread> pool;
  for (unsigned t = 0; t < nth; ++t)
    pool.emplace_back([&, t] {
      long long b_bad = 0, n = 0;
      for (uint32_t mb = t * step; mb < (1u << 23); mb += nth * step) {
        const float b = u2f((127u << 23) | mb);
        const float y = 1.0f / b;
        for (uint32_t ma = 0; ma < 1024; ++ma) {
          const float x = u2f((127u << 23) | (ma << 13));
          b_bad += oxide::exact_div(x, b, y) != x / b;
          ++n;
        }
      }
      bad += b_bad;
      checked += n;
    });
  for (auto& th : pool) th.join();
  CHECK(bad.load() == 0);
  CHECK(checked.load() > 0);
  // Domain edges: exponents of x and b at their limits, both signs, zeros.
  uint64_t rng = 88172645463325252ull;
  for (int i = 0; i < 200000; ++i) {
    rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17;
    const float b = u2f(((127u - 32 + static_cast<uint32_t>(rng % 65)) << 23) | ((rng >> 8) & 0x7fffffu));
    const uint32_t ex = 127u - 60 + static_cast<uint32_t>((rng >> 40) % 125);  // 2^-60 .. 2^64
    float x = u2f((ex << 23) | ((static_cast<uint32_t>(rng >> 32) & 0x3ffu) << 13));
    if (rng & (1ull << 63)) x = -x;
    if (!oxide::exact_div_divisor_ok(b) || !oxide::exact_div_dividend_ok(x)) continue;
    const float y = 1.0f / b;
    CHECK(oxide::exact_div(x, b, y) == x / b);
  }
  for (float b : {0x1p-32f, 1.0f, 3.0f, 0x1p32f}) {
    const float y = 1.0f / b;
    CHECK(std::signbit(oxide::exact_div(-0.0f, b, y)) && oxide::exact_div(-0.0f, b, y) == 0.0f);
    CHECK(!std::signbit(oxide::exact_div(0.0f, b, y)) && oxide::exact_div(0.0f, b, y) == 0.0f);
  }
  CHECK(!oxide::exact_div_divisor_ok(0x1p-33f) && !oxide::exact_div_divisor_ok(INFINITY) &&
        !oxide::exact_div_divisor_ok(NAN));
  CHECK(!oxide::exact_div_dividend_ok(0x1p-61f) && !oxide::exact_div_dividend_ok(NAN));
  std::printf("exact_div: %lld pairs checked\n", static_cast<long long>(checked.load()));
}

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "cpu";
  if (mode == "hash" && argc == 4) {
    const std::string hex = argv[3];
    std::vector<uint8_t> bytes;
    for (std::size_t i = 0; i + 1 < hex.size(); i += 2)
      bytes.push_back(static_cast<uint8_t>(std::strtoul(hex.substr(i, 2).c_str(), nullptr, 16)));
    std::printf("%llu\n", static_cast<unsigned long long>(
                              xxh64(bytes.data(), bytes.size(), std::strtoull(argv[2], nullptr, 10))));
    return 0;
  }
  if (mode == "cpu") {
    test_layout();
    test_metadata();
    test_slot_mapping();
    test_block_pool();
    test_cow();
    test_pool_random_ops();
    test_exact_div(false);
  } else if (mode == "div") {
    test_exact_div(argc > 2 && std::string(argv[2]) == "full");
  } else if (mode == "gpu") {
    test_gpu_append_known_answer();
    test_gpu_cow_all_layers();
    test_gpu_prefill_step();
    test_gpu_decode_step();
    test_gpu_decode_step_shared_prefix();
  } else {
    std::printf("usage: test_host cpu|gpu|div [full]|hash <seed> <hex>\n");
    return 2;
  }
  std::printf("%s: %d failures\n", mode.c_str(), g_failures);
  return g_failures == 0 ? 0 : 1;
}
