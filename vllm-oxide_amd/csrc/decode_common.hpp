// Shared state and helpers of the paged decode passes (paged_decode.hip,
// paged_decode_rows.hip): the launch parameters, sequence lengths, the 16-byte
// non-temporal K/V load, the scalar reads of the block table and the new token's
// slot, and the attended-key prefix sums of windowed batches.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "oxide_common.hpp"

namespace oxide {

struct DecodeParams {
  const void* q;
  const void* k;
  const void* v;
  const uint32_t* cu_seqlens_k;
  const int32_t* block_table;
  float* part_o;    // [B, Hq, max_splits, D]
  float* part_lse;  // [B, Hq, max_splits]
  void* out;        // [B, Hq, D]
  // Fused append (paged_decode_attention_append), null otherwise: the new
  // token's K/V [B, Hkv, D] and its slot per sequence.
  const void* new_k;
  const void* new_v;
  const int64_t* slot_mapping;
  int64_t max_blocks;
  int num_blocks;
  int max_seqlen_k;
  int num_heads;
  int num_kv_heads;
  int block_size;
  int window_left;
  int split_tokens;
  int max_splits;
  int batch;
  int num_wgs;  // balanced paths: key ranges per kv head (persistent, stream, rows)
  int stream_deep;  // stream path: two tiles in flight per wave (see launch_stream)
  float scale_log2;
  // Stream and row paths with a window: prefix sums of the attended keys per
  // sequence (written by pass 1's first workgroup, read by the merge).
  uint32_t* attn_cu;
  // Cascaded call (paged_decode_attention_shared_prefix), null otherwise: the
  // number of leading block-table entries every sequence shares, written by the
  // shared-prefix pass.  The stream pass then attends only keys from
  // shared_blocks[0] * block_size on, writes whole sequences as partials too (at
  // split pre_splits of the prefix rows), and the merge adds the prefix pass's
  // partial rows: row pre_row0 + s * batch * Hq + b * Hq + h for split s.
  const int* shared_blocks;
  int64_t pre_row0;
  int pre_splits;
  int split_keys;
  int64_t whole_row0;  // pre_row0 + pre_splits * batch * Hq; -1 without a cascade
  // Cascaded call: the caller's upper bound on the shared entries (0 otherwise).
  // The stream pass finds the shared count itself (find_shared_blocks, the same
  // function and inputs as the prefix pass), so it need not wait for that pass.
  int shared_hint;
  // Stream pass workgroups (a multiple of 8); 0 = one per CU.  Fewer when the
  // prefix pass of a cascaded call runs beside it on the remaining CUs.
  int stream_wgs;
};

// Shared-prefix pass of a cascaded decode call (paged_prefill.hip): attention of
// every (sequence, query head) row of the decode batch over the leading
// block-table entries all rows share (found on the device, at most shared_hint),
// as partial rows per key split.
struct DecodePrefixArgs {
  const void* q;
  const void* k;
  const void* v;
  const uint32_t* cu_seqlens_k;
  const int32_t* block_table;
  int64_t max_blocks;
  int num_blocks;
  int batch;
  int num_heads;
  int num_kv_heads;
  int head_dim;
  int block_size;
  int max_seqlen_k;
  int window_left;
  float scale_log2;
  float* part_o;
  float* part_lse;
  int64_t pre_row0;
  int pre_splits;
  int split_keys;
  int shared_hint;
  int* shared_out;
  bool bf16;
};
bool launch_decode_prefix(const DecodePrefixArgs& a, hipStream_t s);

// First pass of the row path (paged_decode_rows.hip): launches it for a shape
// rows_path_ok accepts and returns true; p.num_wgs is set to its key ranges.
bool launch_rows_pass1(DecodeParams& p, bool bf16, hipStream_t s);
// Shapes the row path takes: head_dim 128, 8 kv heads, group size 4, and
// power-of-two pages, and batches whose sequence boundaries fit its LDS table.
bool rows_path_ok(int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t block_size);
// Partial rows the row path writes at most (two per range, kv head and query).
int64_t rows_partial_rows(int64_t num_heads);

}  // namespace oxide

namespace {

using oxide::DecodeParams;

constexpr int kXcds = 8;  // MI355X: workgroup i runs on XCD i % 8

// One 16-byte K/V chunk.
// Non-temporal: K/V are streamed once per call (measured on MI355X: plain
// loads cost 4-8 % on every decode path).
__device__ __forceinline__ uint4 load_kv16(const uint16_t* p) {
  const oxide::u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const oxide::u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Keys of sequence b.  Lengths beyond max_seqlen_k (a caller error) are
// clamped so that neither pass can index past the workspace or the block-table
// row; a decreasing cu_seqlens_k reads as an empty sequence.
__device__ __forceinline__ int seq_len(const DecodeParams& p, int b) {
  const int64_t n = static_cast<int64_t>(p.cu_seqlens_k[b + 1]) - p.cu_seqlens_k[b];
  return static_cast<int>(n < 0 ? 0 : (n > p.max_seqlen_k ? p.max_seqlen_k : n));
}

// The block table is not written while a kernel runs.  Read through the
// constant address space (kScalar), wave-uniform lookups compile to scalar
// loads, counted apart from the K/V vector loads, and a wave keeps two tiles in
// flight.  Read as ordinary memory they are vector loads: the lookup for tile
// t + 1, issued after tile t's loads, completes after them (vector loads
// complete in issue order), so tile t + 1's loads wait for tile t and a wave
// keeps one tile in flight -- which the stream pass over long ranges prefers
// (measured on MI355X; see launch_stream).
template <bool kScalar>
struct BtEntry {
  typedef const int32_t type;
};
template <>
struct BtEntry<true> {
  typedef __attribute__((address_space(4))) const int32_t type;
};
// The new token's slot of sequence b (fused append), read through the constant
// address space: a scalar load, so waiting for it does not also wait for the
// K/V tiles in flight (a vector load here took a vmcnt(0) at every owning
// segment's start).
__device__ __forceinline__ int64_t new_token_slot(const DecodeParams& p, int b) {
  typedef __attribute__((address_space(4))) const int64_t slot_t;
  return ((slot_t*)p.slot_mapping)[b];
}

template <bool kScalar>
__device__ __forceinline__ typename BtEntry<kScalar>::type* block_row(const DecodeParams& p, int b) {
  return (typename BtEntry<kScalar>::type*)(p.block_table + static_cast<int64_t>(b) * p.max_blocks);
}

// Cascaded calls: the number of leading block-table entries that are the same
// block ids in every row of the batch, at most hint, and at most
// (L_b - 1) / block_size for every sequence b (so each sequence keeps its newest
// key outside the prefix; an empty sequence makes it 0).  Called by every thread
// of a workgroup of kT threads; the lengths and the table entries are read in
// one round of loads (entries up to hint, within every row since hint <=
// max_blocks) and reduced through one LDS minimum, which every thread returns.
// The prefix pass and the stream pass both call it on the same inputs, so they
// agree on the count without waiting for each other.
template <int kT>
__device__ __forceinline__ int find_shared_blocks(const uint32_t* cu_seqlens_k, const int32_t* block_table,
                                                  int64_t max_blocks, int batch, int block_size, int max_seqlen_k,
                                                  int hint) {
  __shared__ int s_min;
  if (threadIdx.x == 0) s_min = hint;
  __syncthreads();
  int m = hint;
  for (int b = threadIdx.x; b < batch; b += kT) {
    const int64_t n = static_cast<int64_t>(cu_seqlens_k[b + 1]) - cu_seqlens_k[b];
    const int L = static_cast<int>(n < 0 ? 0 : (n > max_seqlen_k ? max_seqlen_k : n));
    m = min(m, L > 0 ? (L - 1) / block_size : 0);
  }
  const int64_t total = static_cast<int64_t>(batch - 1) * hint;
  for (int64_t x = threadIdx.x; x < total; x += kT) {
    const int64_t b = 1 + x / hint;
    const int j = static_cast<int>(x % hint);
    if (block_table[b * max_blocks + j] != block_table[j]) m = min(m, j);
  }
  atomicMin(&s_min, m);
  __syncthreads();
  return s_min;
}

// Largest b in [0, batch) with cu[b] <= key (cu non-decreasing).
__device__ __forceinline__ int find_seq(const uint32_t* cu, int batch, int64_t key) {
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (static_cast<int64_t>(cu[mid]) <= key)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// Windowed (or cascaded) balanced passes: the attended keys of sequence b are
// [lo_b, L_b) with L_b = seq_len, lo_b = max(key_floor, L_b - 1 - window_left)
// (the window term only with a window; lo_b <= L_b); cu[0..batch]
// receives their exclusive prefix sums and lo[b] the lo_b (a workgroup scan in
// LDS: each thread sums a run of sequences, the run totals are scanned, the runs
// written).  Called by every thread of a workgroup of kT threads.
template <int kT>
__device__ __forceinline__ void attended_prefix(const DecodeParams& p, uint32_t* cu, int* lo, int key_floor = 0) {
  __shared__ uint32_t run_sum[kT];
  const int t = threadIdx.x;
  const int per = (p.batch + kT - 1) / kT;
  const int b0 = min(p.batch, t * per), b1 = min(p.batch, b0 + per);
  uint32_t s = 0;
  for (int b = b0; b < b1; ++b) {
    const int L = seq_len(p, b);
    const int l0 = min(L, max(key_floor, p.window_left >= 0 ? L - 1 - p.window_left : 0));
    lo[b] = l0;
    s += static_cast<uint32_t>(L - l0);
  }
  run_sum[t] = s;
  __syncthreads();
  for (int off = 1; off < kT; off <<= 1) {  // inclusive scan of the run totals
    const uint32_t v = t >= off ? run_sum[t - off] : 0u;
    __syncthreads();
    run_sum[t] += v;
    __syncthreads();
  }
  uint32_t x = t > 0 ? run_sum[t - 1] : 0u;
  for (int b = b0; b < b1; ++b) {
    cu[b] = x;
    x += static_cast<uint32_t>(seq_len(p, b) - lo[b]);
  }
  if (t == kT - 1) cu[p.batch] = run_sum[kT - 1];
}

}  // namespace
