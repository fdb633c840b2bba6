// Prefill attention over the paged KV cache (and over contiguous K/V), causal
// with an optional left window and GQA, for gfx950.
//
// What it computes: the seqlen_q >= 1 call of flash_attn_varlen_paged_windowed
// (crates/vllm-oxide/src/attention/flash_attn.rs:52-67) with window_right = 0,
// and, over contiguous K/V, flash_attn_varlen(..., causal = true)
// (flash_attn.rs:15-37, called from the prefill branch of qwen3.rs).  Sequence
// b has Lq = cu_seqlens_q[b+1] - cu_seqlens_q[b] query tokens and
// Lk = cu_seqlens_k[b+1] - cu_seqlens_k[b] keys; the masks are aligned to the
// bottom right (FlashAttention 2): query i, head h sees keys
//     j <= hi = i + Lk - Lq,   j >= hi - window_left (window_left >= 0 only),
// of kv head h / G.  Keys already in the cache before this step (a prefix
// hit, or earlier chunks of a chunked prefill) are simply the first Lk - Lq
// keys, so the paged form needs no gather.  A query with no visible key gets
// zeros.  fp32 accumulation, output rounded to the input dtype once.
//
// Work split: one workgroup of 4 waves per (128 (token, head) rows of one kv
// head's group, kv head, sequence).  Row r of the workgroup is token r / G,
// head r % G of the group, so the G heads that share a kv head share every
// K/V tile.  Each wave owns 32 rows, the 32 columns of its MFMA tiles (lanes l
// and l + 32 share row l % 32).  K/V advance in 64-key tiles loaded straight
// into LDS by the whole workgroup, two LDS buffers (one barrier per tile).
// Per tile and wave, with 32 x 32 x 16 MFMAs (half the issue cost per flop of
// 16 x 16 x 32, so the other wave's softmax work hides behind the matrix pipe):
//   * S^T[key][row] = K . Q^T: A = 32 keys x 16 d from the K tile (XOR-swizzled
//     16-byte chunks), B = the rows' queries, held in registers for the whole
//     kernel.  Lane l gets keys 8(r/4) + 4(l/32) + r%4 of each 32-key block.
//   * online softmax per row in the log2 domain; a row's keys sit in lanes l
//     and l ^ 32, so the maximum takes one v_permlane32_swap and the sums stay
//     per lane until the end.
//   * O^T[d][row] += V^T . P^T: A = V^T from two transposing LDS reads of the
//     row-major V tile (keys 16s + 4(l/32) + 0..3 and + 8 of a 32-key block),
//     B = the lane's own probabilities in the same key order (registers
//     8s..8s+7 of the score block), so P never moves between lanes.  Every
//     accumulator of a lane belongs to its own row: rescaling is a per-lane
//     multiply.
// Workgroup order is XCD-aware: all row tiles of one (sequence, kv head) run
// on one XCD (workgroup i runs on XCD i % 8), so its K/V is fetched from HBM
// once into that XCD's L2 and re-read from there; within a unit the tiles
// with the most keys (last tokens) start first.  For short prompts (kPair) a
// workgroup takes two row tiles of its unit, n - 1 - i and then i.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "cdna4_tile.hpp"
#include "decode_common.hpp"
#include "oxide_common.hpp"

namespace {

constexpr int kPfWaves = 4;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfRows = kPfWaves * 32;  // (token, head) rows per workgroup
constexpr int kPfKeys = 64;             // keys per K/V tile
constexpr int kPfXcds = 8;

struct PrefillParams {
  const void* q;    // [total_q, Hq, D]
  const void* k;    // paged [NB, BS, Hkv, D] or contiguous [total_k, Hkv, D]
  const void* v;
  void* out;        // [total_q, Hq, D]
  const uint32_t* cu_seqlens_q;
  const uint32_t* cu_seqlens_k;
  const int32_t* block_table;  // null: contiguous K/V, key j of b at row cu_seqlens_k[b] + j
  int64_t max_blocks;
  int64_t num_rows;            // rows of the K/V view (clamp for bad indices)
  int num_blocks;
  int max_seqlen_q;
  int max_seqlen_k;
  int num_heads;
  int num_kv_heads;
  int group;
  int tokens_per_wg;
  int tiles_per_unit;
  int units;                   // batch * num_kv_heads
  int block_size;
  int window_left;
  float scale_log2;
  // Shared-prefix pass of a decode batch (kernel instances with kPrefix): the rows
  // are the decode batch's (sequence, query head) pairs -- q [dec_batch, Hq, D],
  // cu_seqlens_k the decode batch's -- and the keys are the leading block-table
  // entries that every row shares (at most shared_hint of them; the kernel finds
  // how many), cut into pre_splits splits of split_keys keys.  Each (split,
  // sequence, head) writes a normalised partial row and its log2-sum-exp at row
  // pre_row0 + split * dec_batch * Hq + b * Hq + h of part_o / part_lse.
  float* part_o;
  float* part_lse;
  int64_t pre_row0;
  int pre_splits;
  int split_keys;
  int shared_hint;
  int dec_batch;
  int* shared_out;  // the number of shared blocks found (written by workgroup 0)
  int pair;         // 1: each workgroup takes row tiles n - 1 - i and then i of its unit
};

__device__ __forceinline__ int clamp_len(int64_t n, int cap) {
  return static_cast<int>(n < 0 ? 0 : (n > cap ? cap : n));
}

// LDS tile layouts (64 keys, row = one key's head slice of 2*D bytes):
//   K: 16-byte chunk c of row r at chunk position c ^ kswz(r).  One MFMA
//      operand read (16 lanes = 16 consecutive rows, one chunk each) then
//      covers all 64 banks: rows are 256 B apart at D = 128 (kswz = r % 16);
//      at D = 64 rows r and r + 1 sit in opposite bank halves and
//      kswz = (r >> 1) % 8 separates the 8 pairs.
//   V: 32-byte granule g of row r at granule position g ^ vswz(r).  One
//      transposing read covers 4 consecutive rows x 2 adjacent granules per
//      half-wave; vswz = 2 (r % 4) at D = 128 (and r & 2 at D = 64, where
//      odd rows add half a bank sweep) maps those 8 pieces to distinct banks.
// Both are written by direct global -> LDS loads (global_load_lds_dwordx4):
// lane i of a wave instruction fills bytes [16 i, 16 i + 16) of a 1 KiB run,
// so each lane loads the source chunk that belongs at its LDS position.
template <int D>
__device__ __forceinline__ int kswz(int r) {
  return D == 128 ? (r & 15) : ((r >> 1) & 7);
}
template <int D>
__device__ __forceinline__ int vswz(int r) {
  return D == 128 ? 2 * (r & 3) : (r & 2);
}

// One direct global -> LDS load of 16 bytes per lane: lane i writes LDS bytes
// [lds + 16 i, lds + 16 i + 16).  Issued as inline assembly so the compiler
// does not treat the in-flight loads as possibly aliasing the other buffer's
// LDS reads (it otherwise waits for them before some transposing reads); the
// kernel waits for them itself (vmcnt(0) before the barrier that publishes
// the tile).  `lds` must be wave-uniform.
__device__ __forceinline__ void load_lds16(const void* src, const char* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(src)
               : "memory", "m0");
}
// The same from a wave-uniform base address plus a 32-bit per-lane byte offset.
__device__ __forceinline__ void load_lds16(const void* base, uint32_t voff, const char* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0), "v"(voff), "s"(base)
               : "memory", "m0");
}

// K/V addressing of a kernel instance.
enum PrefillAddressing {
  kContiguous = 0,  // key j of sequence b at row cu_seqlens_k[b] + j
  kPagedTiles = 1,  // paged, block_size a multiple of the 64-key tile: one block per tile
  kPagedRows = 2,   // paged, any block_size: a block lookup per row
};

template <class Tag, int D, int MODE, bool kPrefix, bool kPair = false>
__global__ __launch_bounds__(kPfThreads, 2) void paged_prefill_attn(PrefillParams p) {
  constexpr int CH = D / 8;                  // 16-byte chunks per head row
  constexpr int KS = D / 16;                 // MFMA k-steps of Q.K (16 dims each)
  constexpr int NDB = D / 32;                // 32-wide d blocks of O (two 32-byte V granules)
  constexpr int ROWB = 2 * D;                // bytes per tile row
  constexpr int TBYTES = kPfKeys * ROWB;     // one K or V tile
  constexpr int BUF = 2 * TBYTES;            // K tile | V tile
  constexpr int RPI = 1024 / ROWB;           // tile rows per wave load instruction
  constexpr int WROWS = kPfKeys / kPfWaves;  // tile rows loaded by each wave
  constexpr int NLD = WROWS / RPI;           // load instructions per wave and tensor
  static_assert(WROWS % RPI == 0, "tile rows");
  // Two LDS buffers as separate objects: the loop is unrolled by two so each
  // access names its buffer statically, which lets the compiler see that the
  // loads in flight into one buffer do not alias reads of the other.
  __shared__ __align__(1024) char smem0[BUF];
  __shared__ __align__(1024) char smem1[BUF];

  // XCD-aware work item: unit (sequence, kv head) u sits on XCD u % 8 and its
  // tiles are consecutive workgroups there, heaviest first.  Shared-prefix pass:
  // unit (key split, kv head), all of them over table row 0 (the shared entries).
  const int i = blockIdx.x;
  const int j = i / kPfXcds;
  const int wpu = kPair ? (p.tiles_per_unit + 1) / 2 : p.tiles_per_unit;  // workgroups per unit
  const int u = (j / wpu) * kPfXcds + i % kPfXcds;
  if (u >= p.units) return;
  const int jj = j % wpu;
  for (int pass = 0; pass < (kPair ? 2 : 1); ++pass) {
  const int tile = pass == 0 ? p.tiles_per_unit - 1 - jj : jj;
  if (pass == 1) {
    if (tile >= p.tiles_per_unit - 1 - jj) break;  // the middle tile of an odd count: done
    __syncthreads();  // the previous tile's last LDS reads before this tile's first loads
  }
  const int b = kPrefix ? 0 : u / p.num_kv_heads;
  const int kh = u % p.num_kv_heads;
  const int split = kPrefix ? u / p.num_kv_heads : 0;

  int Lq, Lk;
  if constexpr (kPrefix) {
    const int shared = find_shared_blocks<kPfThreads>(p.cu_seqlens_k, p.block_table, p.max_blocks, p.dec_batch,
                                                      p.block_size, p.max_seqlen_k, p.shared_hint);
    if (blockIdx.x == 0 && threadIdx.x == 0) *p.shared_out = shared;
    Lq = p.dec_batch;
    Lk = shared * p.block_size;  // the shared keys; no sequence attends past them here
    if (split * p.split_keys >= Lk) continue;
  } else {
    Lq = clamp_len(static_cast<int64_t>(p.cu_seqlens_q[b + 1]) - p.cu_seqlens_q[b], p.max_seqlen_q);
    Lk = clamp_len(static_cast<int64_t>(p.cu_seqlens_k[b + 1]) - p.cu_seqlens_k[b], p.max_seqlen_k);
  }
  const int t0 = tile * p.tokens_per_wg;
  if (t0 >= Lq) continue;
  const int t1 = min(Lq, t0 + p.tokens_per_wg);
  const int off = Lk - Lq;  // hi of token t is t + off
  const int G = p.group;
  const int W = p.window_left;

  // Key range of the workgroup: [klo, khi] (empty when khi < klo).  Shared-prefix
  // pass: the split's keys, every row seeing all of them but those before its window.
  const int khi = kPrefix ? min(Lk, (split + 1) * p.split_keys) - 1 : min(Lk - 1, t1 - 1 + off);
  const int klo = kPrefix ? split * p.split_keys : (W >= 0 ? max(0, t0 + off - W) : 0);
  const int kt0 = klo & ~(kPfKeys - 1);
  const int ntiles = khi >= klo ? (khi - kt0) / kPfKeys + 1 : 0;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t q0 = kPrefix ? 0 : p.cu_seqlens_q[b];
  const int rows_used = p.tokens_per_wg * G;

  // This lane's row (column l % 32 of the MFMA tiles; lanes l and l + 32 share
  // it and hold alternate groups of four keys): token, head, key range.
  const int r32 = lane & 31;
  const int half = lane >> 5;
  const int rr = wave * 32 + r32;
  const int tq = t0 + rr / G;
  const bool valid = rr < rows_used && tq < t1;
  const int64_t qrow = valid ? (q0 + tq) * p.num_heads + kh * G + rr % G : 0;
  int hi_r = valid ? tq + off : -1;
  int lo_r = valid && W >= 0 ? tq + off - W : 0;
  if constexpr (kPrefix) {
    // Decode sequence tq attends keys [max(0, L - 1 - W), L) of which the shared
    // ones are [.., Lk); this split holds [klo, khi].
    const int L = valid ? clamp_len(static_cast<int64_t>(p.cu_seqlens_k[tq + 1]) - p.cu_seqlens_k[tq],
                                    p.max_seqlen_k)
                        : 0;
    hi_r = valid ? khi : -1;
    lo_r = valid && W >= 0 ? L - 1 - W : 0;
  }
  // Key range of the wave's valid rows (wave-uniform) for skipping tiles.
  const int wr0 = wave * 32;
  const int wt_first = t0 + wr0 / G;
  const int wt_last = min(t1 - 1, t0 + min(wr0 + 31, rows_used - 1) / G);
  const bool wave_active = wr0 < rows_used && wt_first < t1;
  const int wave_hi = kPrefix ? khi : min(Lk - 1, wt_last + off);
  const int wave_lo = kPrefix ? 0 : (W >= 0 ? wt_first + off - W : 0);

  // Queries (B operand of S^T, 16 dims per k-step).  A negative scale is
  // applied as a sign flip of q (exact) and |scale|, so the running maxima can
  // be taken on raw scores.
  const uint32_t qflip = p.scale_log2 < 0.f ? 0x80008000u : 0u;
  const float c_log2 = fabsf(p.scale_log2);
  uint4 qb[KS];  // loaded after the first tile's loads are issued

  // Direct tile loads: wave w fills tile rows [16 w, 16 w + 16); lane -> (row
  // within the 1 KiB run, 16-byte position), source chunk chosen by the swizzle.
  const int lrow = lane / CH;         // row within the run
  const int lpos = lane % CH;         // 16-byte position within the row
  const int64_t row_stride = static_cast<int64_t>(p.num_kv_heads) * D;
  const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + kh * D;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + kh * D;
  const int32_t* bt = p.block_table + (MODE == kContiguous ? 0 : b * p.max_blocks);
  const int64_t kstart = p.cu_seqlens_k[b];
  // Per-lane constants: tile row of each load, its byte offset in the tile's
  // source rows, and the swizzled source chunks.
  int trow[NLD];
  uint32_t koff[NLD], voff[NLD], kchb[NLD], vchb[NLD];
  int blk_next[NLD];
#pragma unroll
  for (int x = 0; x < NLD; ++x) {
    trow[x] = wave * WROWS + x * RPI + lrow;
    kchb[x] = 16 * (lpos ^ kswz<D>(trow[x]));
    vchb[x] = 32 * ((lpos >> 1) ^ vswz<D>(trow[x])) + 16 * (lpos & 1);
    koff[x] = static_cast<uint32_t>(trow[x] * row_stride * 2) + kchb[x];
    voff[x] = static_cast<uint32_t>(trow[x] * row_stride * 2) + vchb[x];
    blk_next[x] = 0;
  }
  // Block-table entries of the tile at kb0 (one per tile, or one per row),
  // read a tile ahead of its loads so their latency hides behind a tile of math.
  auto fetch_blocks = [&](int kb0) {
    if (MODE == kPagedTiles) {
      blk_next[0] = bt[kb0 / p.block_size];
    } else if (MODE == kPagedRows) {
#pragma unroll
      for (int x = 0; x < NLD; ++x) blk_next[x] = bt[min(kb0 + trow[x], Lk - 1) / p.block_size];
    }
  };
  auto issue_tile = [&](int kb0, char* sbuf) {
    if (MODE == kPagedRows) {
      // General pages: a 64-bit source address per lane.
      int64_t rows[NLD];
#pragma unroll
      for (int x = 0; x < NLD; ++x) {
        const int key = min(kb0 + trow[x], Lk - 1);
        const int blk = min(max(blk_next[x], 0), p.num_blocks - 1);
        rows[x] = static_cast<int64_t>(blk) * p.block_size + key % p.block_size;
      }
#pragma unroll
      for (int x = 0; x < NLD; ++x) {
        char* dst = sbuf + (wave * WROWS + x * RPI) * ROWB;
        load_lds16(kbase + rows[x] * row_stride + kchb[x] / 2, dst);
        load_lds16(vbase + rows[x] * row_stride + vchb[x] / 2, dst + TBYTES);
      }
    } else {
      // The tile's rows are consecutive: a uniform base row plus per-lane
      // offsets; rows past the last valid one repeat it.
      int64_t row0;
      int lim;  // last valid tile row
      if (MODE == kPagedTiles) {
        const int blk = min(max(__builtin_amdgcn_readfirstlane(blk_next[0]), 0), p.num_blocks - 1);
        row0 = static_cast<int64_t>(blk) * p.block_size + kb0 % p.block_size;
        lim = Lk - 1 - kb0;
      } else {
        row0 = min(kstart + kb0, p.num_rows - 1);
        lim = static_cast<int>(min<int64_t>(Lk - 1 - kb0, p.num_rows - 1 - row0));
      }
      const uint32_t limb = static_cast<uint32_t>(lim * row_stride * 2);
      const uint16_t* kt = kbase + row0 * row_stride;
      const uint16_t* vt = vbase + row0 * row_stride;
#pragma unroll
      for (int x = 0; x < NLD; ++x) {
        const bool in = trow[x] <= lim;
        char* dst = sbuf + (wave * WROWS + x * RPI) * ROWB;
        load_lds16(kt, in ? koff[x] : limb + kchb[x], dst);
        load_lds16(vt, in ? voff[x] : limb + vchb[x], dst + TBYTES);
      }
    }
  };

  float m_r = -INFINITY;  // running max of raw scores (x |scale| log2 e)
  // Row sum of the probabilities as rounded for the P.V product (packed
  // pairs summed by v_dot2c), over this lane's half of the keys.
  float lsum = 0.f;
  floatx16 acc[NDB];
#pragma unroll
  for (int r = 0; r < 16; ++r)
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[db][r] = 0.f;

  auto step = [&](int it, char* cur, char* nxt) {
    const int kb0 = kt0 + it * kPfKeys;
    // Tile it has landed in LDS (own loads, then everyone's); then start the
    // next tile into the other buffer, whose readers finished before this barrier.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (it + 1 < ntiles) issue_tile(kb0 + kPfKeys, nxt);
    if (wave_active && kb0 <= wave_hi && kb0 + kPfKeys - 1 >= wave_lo) {
      const uint4* sk = reinterpret_cast<const uint4*>(cur);
      const char* sv = cur + TBYTES;

      // S^T of two 32-key blocks: lane l holds keys 8 (r / 4) + 4 half + r % 4
      // of block kb for its row.
      floatx16 sc[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[kb][r] = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const uint4 ka = sk[(kb * 32 + r32) * CH + ((2 * ks + half) ^ kswz<D>(r32))];
          sc[kb] = mfma32x32x16(Tag{}, ka, qb[ks], sc[kb]);
        }
      }

      // Mask only where the tile crosses some row's key range.
      const bool lane_mask = !(kb0 >= lo_r && kb0 + kPfKeys - 1 <= hi_r);
      if (__ballot(lane_mask) != 0) {
        const int k0 = kb0 + 4 * half;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = k0 + kb * 32 + 8 * (r / 4) + r % 4;
            sc[kb][r] = (key > hi_r || key < lo_r) ? -INFINITY : sc[kb][r];
          }
      }
      float mt = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sc[kb][r]);
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
        const float a = __uint_as_float(sw[0]), b = __uint_as_float(sw[1]);
        mt = a > b ? a : b;
      }
      // Lazy rescaling: keep the old maximum while the tile's stays within
      // 2^8 of it (probabilities <= 256, exact in fp32 and bf16 range), so
      // most tiles skip the accumulator multiplies.
      const float ms = mt * c_log2;
      const bool grow = ms > m_r + 8.f;
      float alpha = 1.f;
      if (grow) {
        alpha = __builtin_amdgcn_exp2f(m_r - ms);
        m_r = ms;
      }
      if (__ballot(grow) != 0) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[db] *= alpha;
        lsum *= alpha;
      }
      const float msafe = m_r == -INFINITY ? 0.f : m_r;

      // P^T: the 8 registers 8 s .. 8 s + 7 of block kb are the B operand of
      // k-step (kb, s), keys kb * 32 + 16 s + 4 half + {0..3} and + 8 + {0..3}.
      uint4 pb[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float x[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kb][r], c_log2, -msafe));
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          pb[kb][s2].x = pack2(Tag{}, x[8 * s2 + 0], x[8 * s2 + 1]);
          pb[kb][s2].y = pack2(Tag{}, x[8 * s2 + 2], x[8 * s2 + 3]);
          pb[kb][s2].z = pack2(Tag{}, x[8 * s2 + 4], x[8 * s2 + 5]);
          pb[kb][s2].w = pack2(Tag{}, x[8 * s2 + 6], x[8 * s2 + 7]);
          lsum = sum2_acc(Tag{}, pb[kb][s2].x, lsum);
          lsum = sum2_acc(Tag{}, pb[kb][s2].y, lsum);
          lsum = sum2_acc(Tag{}, pb[kb][s2].z, lsum);
          lsum = sum2_acc(Tag{}, pb[kb][s2].w, lsum);
        }
      }

      // O^T += V^T . P^T: the A operand of d block db for k-step (kb, s) is two
      // transposing reads; lane i of 16-lane group g reads key row
      // kb * 32 + 16 s + 4 half + i / 4 (and + 8), 4 dims at
      // 32 db + 16 (g % 2) + 4 (i % 4), i.e. granule 2 db + g % 2.
      const int gsub = (lane >> 4) & 1;
      const int i16 = lane & 15;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int rlo = kb * 32 + 16 * s2 + 4 * half + i16 / 4;
          const char* vlo = sv + rlo * ROWB + 8 * (i16 % 4);
          const char* vhi = vlo + 8 * ROWB;
          const int zlo = vswz<D>(rlo), zhi = vswz<D>(rlo + 8);
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const int g = 2 * db + gsub;
            const uint2 a0 = lds_read_tr16(vlo + 32 * (g ^ zlo));
            const uint2 a1 = lds_read_tr16(vhi + 32 * (g ^ zhi));
            const uint4 va = make_uint4(a0.x, a0.y, a1.x, a1.y);
            acc[db] = mfma32x32x16(Tag{}, va, pb[kb][s2], acc[db]);
          }
        }
    }
    // Block-table entries for the tile after next, once this tile's LDS reads
    // are issued (they complete under the next barrier's wait).
    if (it + 2 < ntiles) fetch_blocks(kb0 + 2 * kPfKeys);
  };
  if (ntiles > 0) {
    fetch_blocks(kt0);
    issue_tile(kt0, smem0);
    if (ntiles > 1) fetch_blocks(kt0 + kPfKeys);
  }
  // The queries load while the first tile is in flight: k-step ks takes dims
  // 16 ks + 8 half .. + 7.
  {
    const uint16_t* qp = static_cast<const uint16_t*>(p.q) + qrow * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint4 v = valid ? *reinterpret_cast<const uint4*>(qp + 16 * ks + 8 * half) : make_uint4(0, 0, 0, 0);
      v.x ^= qflip; v.y ^= qflip; v.z ^= qflip; v.w ^= qflip;
      qb[ks] = v;
    }
  }

  for (int it = 0; it < ntiles; it += 2) {
    step(it, smem0, smem1);
    if (it + 1 < ntiles) step(it + 1, smem1, smem0);
  }

  // out[row][d] for d = 32 db + 8 q + 4 half + e (register 4 q + e), normalised
  // by the row total (both halves of the keys).
  lsum = sum_over_halves(lsum);
  if (kPrefix && valid) {
    // Normalised partial row and its log2-sum-exp (scores are in units of
    // |scale| log2 e, as the decode passes' partials).
    const float l = lsum;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int64_t prow = p.pre_row0 + static_cast<int64_t>(split) * p.dec_batch * p.num_heads + qrow;
    float* po = p.part_o + prow * D + 4 * half;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4*>(po + 32 * db + 8 * q) =
            make_float4(acc[db][4 * q + 0] * inv, acc[db][4 * q + 1] * inv, acc[db][4 * q + 2] * inv,
                        acc[db][4 * q + 3] * inv);
    if (half == 0) p.part_lse[prow] = l > 0.f ? m_r + log2f(l) : -INFINITY;
  } else if (valid) {
    const float l = lsum;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t* op = static_cast<uint16_t*>(p.out) + qrow * D + 4 * half;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint2 w;
        w.x = pack2(Tag{}, acc[db][4 * q + 0] * inv, acc[db][4 * q + 1] * inv);
        w.y = pack2(Tag{}, acc[db][4 * q + 2] * inv, acc[db][4 * q + 3] * inv);
        *reinterpret_cast<uint2*>(op + 32 * db + 8 * q) = w;
      }
  }
  }
}

int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

template <class Tag, int D>
void launch_mode(const PrefillParams& p, dim3 grid, hipStream_t s) {
  if (p.pair) {
    if (p.block_table == nullptr)
      hipLaunchKernelGGL((paged_prefill_attn<Tag, D, kContiguous, false, true>), grid, dim3(kPfThreads), 0, s, p);
    else if (p.block_size % kPfKeys == 0)
      hipLaunchKernelGGL((paged_prefill_attn<Tag, D, kPagedTiles, false, true>), grid, dim3(kPfThreads), 0, s, p);
    else
      hipLaunchKernelGGL((paged_prefill_attn<Tag, D, kPagedRows, false, true>), grid, dim3(kPfThreads), 0, s, p);
    return;
  }
  if (p.block_table == nullptr)
    hipLaunchKernelGGL((paged_prefill_attn<Tag, D, kContiguous, false>), grid, dim3(kPfThreads), 0, s, p);
  else if (p.block_size % kPfKeys == 0)
    hipLaunchKernelGGL((paged_prefill_attn<Tag, D, kPagedTiles, false>), grid, dim3(kPfThreads), 0, s, p);
  else
    hipLaunchKernelGGL((paged_prefill_attn<Tag, D, kPagedRows, false>), grid, dim3(kPfThreads), 0, s, p);
}

template <class Tag, int D>
void launch_prefix_mode(const PrefillParams& p, dim3 grid, hipStream_t s) {
  if (p.block_size % kPfKeys == 0)
    hipLaunchKernelGGL((paged_prefill_attn<Tag, D, kPagedTiles, true>), grid, dim3(kPfThreads), 0, s, p);
  else
    hipLaunchKernelGGL((paged_prefill_attn<Tag, D, kPagedRows, true>), grid, dim3(kPfThreads), 0, s, p);
}

template <class Tag>
bool launch_prefill(const PrefillParams& p, int head_dim, hipStream_t s) {
  const int64_t units8 = ceil_div64(p.units, kPfXcds) * kPfXcds;
  const dim3 grid(static_cast<unsigned>(units8 * (p.pair ? (p.tiles_per_unit + 1) / 2 : p.tiles_per_unit)));
  if (head_dim == 128) {
    launch_mode<Tag, 128>(p, grid, s);
    return true;
  }
  if (head_dim == 64) {
    launch_mode<Tag, 64>(p, grid, s);
    return true;
  }
  return false;
}

void prefill_impl(void* out, const void* q, const void* k, const void* v, const uint32_t* cu_seqlens_q,
                  const uint32_t* cu_seqlens_k, const int32_t* block_table, int64_t max_blocks_per_seq,
                  int64_t num_blocks, int64_t num_rows, int64_t batch, int64_t num_heads,
                  int64_t num_kv_heads, int64_t head_dim, int64_t page_block_size,
                  int64_t max_seqlen_q, int64_t max_seqlen_k, int32_t window_left,
                  float softmax_scale, int dtype, void* stream) {
  if (dtype != OXIDE_DTYPE_BF16 && dtype != OXIDE_DTYPE_F16) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_DTYPE);
    return;
  }
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      max_seqlen_q < 0 || max_seqlen_k < 0 || batch > 65535 || num_heads > 65535 ||
      max_seqlen_q > INT32_MAX / 2 || max_seqlen_k > INT32_MAX / 2) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  if (batch == 0 || max_seqlen_q == 0) return;
  if (!out || !q || !cu_seqlens_q || !cu_seqlens_k || !oxide::aligned16(out) || !oxide::aligned16(q)) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  if (max_seqlen_k > 0) {
    if (!k || !v || !oxide::aligned16(k) || !oxide::aligned16(v)) {
      oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
      return;
    }
    if (block_table != nullptr) {
      if (page_block_size <= 0 || num_blocks <= 0 || num_blocks > INT32_MAX || max_blocks_per_seq < 0 ||
          page_block_size > INT32_MAX || max_blocks_per_seq * page_block_size < max_seqlen_k) {
        oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
        return;
      }
    } else if (num_rows <= 0) {
      oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
      return;
    }
  }
  const int64_t group = num_heads / num_kv_heads;
  if ((head_dim != 64 && head_dim != 128) || group > kPfRows) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_SHAPE);
    return;
  }
  PrefillParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.out = out;
  p.cu_seqlens_q = cu_seqlens_q;
  p.cu_seqlens_k = cu_seqlens_k;
  p.block_table = block_table;
  p.max_blocks = max_blocks_per_seq;
  p.num_rows = block_table ? num_blocks * page_block_size : num_rows;
  p.num_blocks = static_cast<int>(block_table ? num_blocks : 0);
  p.max_seqlen_q = static_cast<int>(max_seqlen_q);
  p.max_seqlen_k = static_cast<int>(max_seqlen_k);
  p.num_heads = static_cast<int>(num_heads);
  p.num_kv_heads = static_cast<int>(num_kv_heads);
  p.group = static_cast<int>(group);
  p.tokens_per_wg = static_cast<int>(kPfRows / group);
  const int64_t tiles = ceil_div64(max_seqlen_q, p.tokens_per_wg);
  const int64_t units = batch * num_kv_heads;
  if (units > INT32_MAX / 2 || ceil_div64(units, kPfXcds) * kPfXcds * tiles > INT32_MAX) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  p.tiles_per_unit = static_cast<int>(tiles);
  p.units = static_cast<int>(units);
  // Short prompts with no cached prefix: a workgroup takes a unit's row tiles n - 1 - i
  // and then i (a separate kernel instance), the same keys per workgroup and half the
  // workgroup starts.  Measured on MI355X, Qwen3-8B heads, bit-identical output:
  // 16 x 1024 212.1 -> 202.8 us, 32 x 512 138.6 -> 135.7 us, 8 x 2048 324.2 -> 319.9 us;
  // for 4 x 4096 and 1 x 8192 pairing measured +0.7 / +1.3 %, and with a cached prefix
  // the tiles already carry equal keys.
  p.pair = (tiles >= 2 && max_seqlen_k <= max_seqlen_q && max_seqlen_q <= 2048) ? 1 : 0;
  p.block_size = static_cast<int>(block_table ? page_block_size : 1);
  p.window_left = window_left < 0 ? -1 : window_left;
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  hipStream_t s = oxide::as_stream(stream);
  const bool ok = dtype == OXIDE_DTYPE_BF16 ? launch_prefill<Bf16Tag>(p, static_cast<int>(head_dim), s)
                                            : launch_prefill<F16Tag>(p, static_cast<int>(head_dim), s);
  if (!ok) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_SHAPE);
    return;
  }
  oxide::check_launch();
}

}  // namespace

extern "C" void paged_prefill_attention(void* out, const void* q, const void* k_cache,
                                        const void* v_cache, const uint32_t* cu_seqlens_q,
                                        const uint32_t* cu_seqlens_k, const int32_t* block_table,
                                        int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch,
                                        int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                        int64_t page_block_size, int64_t max_seqlen_q,
                                        int64_t max_seqlen_k, int32_t window_left,
                                        float softmax_scale, int dtype, void* stream) {
  if (block_table == nullptr && max_seqlen_k > 0) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  prefill_impl(out, q, k_cache, v_cache, cu_seqlens_q, cu_seqlens_k, block_table, max_blocks_per_seq,
               num_blocks, 0, batch, num_heads, num_kv_heads, head_dim, page_block_size, max_seqlen_q,
               max_seqlen_k, window_left, softmax_scale, dtype, stream);
}

extern "C" void varlen_prefill_attention(void* out, const void* q, const void* k, const void* v,
                                         const uint32_t* cu_seqlens_q, const uint32_t* cu_seqlens_k,
                                         int64_t total_k, int64_t batch, int64_t num_heads,
                                         int64_t num_kv_heads, int64_t head_dim, int64_t max_seqlen_q,
                                         int64_t max_seqlen_k, int32_t window_left, float softmax_scale,
                                         int dtype, void* stream) {
  prefill_impl(out, q, k, v, cu_seqlens_q, cu_seqlens_k, nullptr, 0, 0, total_k, batch, num_heads,
               num_kv_heads, head_dim, 1, max_seqlen_q, max_seqlen_k, window_left, softmax_scale,
               dtype, stream);
}

namespace oxide {

// Shared-prefix pass of a cascaded decode call (declared in decode_common.hpp).
bool launch_decode_prefix(const DecodePrefixArgs& a, hipStream_t s) {
  PrefillParams p{};
  p.q = a.q;
  p.k = a.k;
  p.v = a.v;
  p.cu_seqlens_k = a.cu_seqlens_k;
  p.block_table = a.block_table;
  p.max_blocks = a.max_blocks;
  p.num_blocks = a.num_blocks;
  p.num_rows = static_cast<int64_t>(a.num_blocks) * a.block_size;
  p.max_seqlen_k = a.max_seqlen_k;
  p.num_heads = a.num_heads;
  p.num_kv_heads = a.num_kv_heads;
  p.group = a.num_heads / a.num_kv_heads;
  p.tokens_per_wg = kPfRows / p.group;
  p.tiles_per_unit = static_cast<int>(ceil_div64(a.batch, p.tokens_per_wg));
  p.units = a.num_kv_heads * a.pre_splits;
  p.block_size = a.block_size;
  p.window_left = a.window_left < 0 ? -1 : a.window_left;
  p.scale_log2 = a.scale_log2;
  p.part_o = a.part_o;
  p.part_lse = a.part_lse;
  p.pre_row0 = a.pre_row0;
  p.pre_splits = a.pre_splits;
  p.split_keys = a.split_keys;
  p.shared_hint = a.shared_hint;
  p.dec_batch = a.batch;
  p.shared_out = a.shared_out;
  const dim3 grid(static_cast<unsigned>(ceil_div64(p.units, kPfXcds) * kPfXcds * p.tiles_per_unit));
  if (a.head_dim == 128) {
    a.bf16 ? launch_prefix_mode<Bf16Tag, 128>(p, grid, s) : launch_prefix_mode<F16Tag, 128>(p, grid, s);
    return true;
  }
  if (a.head_dim == 64) {
    a.bf16 ? launch_prefix_mode<Bf16Tag, 64>(p, grid, s) : launch_prefix_mode<F16Tag, 64>(p, grid, s);
    return true;
  }
  return false;
}

}  // namespace oxide
