// Paged decode attention with GQA, optional left window and split-KV
// (flash-decoding), for gfx950.
//
// What it computes (the decode call of flash_attn_varlen_paged_windowed at
// crates/vllm-oxide/src/attention/flash_attn.rs:52-67, with window_right =
// Some(0) and seqlen_q = 1): for sequence b with L = cu_seqlens_k[b+1] -
// cu_seqlens_k[b] keys and query head h reading kv head h / G,
//     out[b,h,:] = sum_j softmax_j(scale * q[b,h,:] . K_j) V_j,
//     j in [lo, L), lo = max(0, L - 1 - window_left) (0 when window_left < 0),
// where key j lives at row block_table[b][j / BS] * BS + j % BS of the cache
// view [num_blocks, BS, Hkv, D].  Accumulation is fp32; the output is rounded
// to the cache dtype once.
//
// Three interchangeable first passes, chosen by shape (choose_path), share the
// per-wave tile code below:
//   * paged_decode_stream (long batches): 8-wave workgroups, one per CU, wave
//     i on kv head i % Hkv, each streaming an equal range of the batch's keys
//     (with a window, of its attended keys) of its head with no barrier; the
//     pieces of a sequence that crosses ranges merge in
//     paged_decode_merge_stream.
//   * paged_decode_split (short ones): a workgroup per (split, kv head,
//     sequence), merged by paged_decode_merge.
//   * paged_decode_persistent (kv head counts that do not divide 8, long
//     contexts): a workgroup per resident slot over the (sequence, kv head,
//     key) positions, merged by paged_decode_merge_persistent.
//
// Pass 1 of the split grid (paged_decode_split): one workgroup of 4 waves per
// (split, kv head, sequence); a split is 128, 256, 512 or 1024 consecutive logical
// keys (choose_split_tokens), a quarter per wave, walked as 16-key tiles in
// straight-line code with a register double buffer (tile t+1's loads are in
// flight while tile t computes; loads past the wave's last key are clamped to
// a fetched tile and masked).
//   * K and V rows are loaded as whole 256-byte head rows per 16 lanes, four
//     rows per instruction, with non-temporal hints: the shape that streams at
//     full HBM rate.  K is transposed through a wave-private LDS tile into the
//     MFMA layout; V rows are staged in LDS for the transposing reads.
//   * S^T = K . Q^T and O += P . V both on the matrix cores
//     (v_mfma_f32_16x16x32_{bf16,f16}); the tile math is described above
//     paged_decode_split below.
//   * online softmax per query in the log2 domain (scale folded with log2 e).
//   The 4 waves are merged through LDS; a sequence with a single split writes
//   its output directly, otherwise the split writes its normalised partial
//   output o (fp32, [B, Hq, max_splits, D]) and log2-sum-exp.
// Workgroup order is XCD-aware (decode_work_item).
// With the fused append (paged_decode_attention_append) the workgroup whose
// keys include position L-1 first writes its kv head's slice of the new
// token's K/V to slot_mapping[b] and uses those values for that key.
// Pass 2 (paged_decode_merge): 4 waves per (query head, sequence) merge the
// splits that intersect [lo, L) with log-sum-exp weights and write out.
//
// Every path reads K/V exactly once; the partials add 2 * Hq * (D+1) * 4 bytes
// per split or piece (under 1 % at split_tokens = 1024; 1.8 % of the bytes on
// the stream path at Qwen3-8B B=64 ctx 2k-8k).
#include <math.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "cdna4_tile.hpp"
#include "decode_common.hpp"
#include "oxide_common.hpp"

namespace {


constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

// Work item (split, kv head, sequence) of this workgroup; false for padding.
// 1-D grid, XCD-grouped: a unit u = (seq, split) is pinned to XCD u % 8 and its
// kv heads are consecutive workgroups there, so one XCD reads all head slices
// of the unit's token rows together.  Units are numbered split-major with the
// sequence rotated by the split index, so consecutive splits of one sequence
// land on different XCDs and ragged lengths spread evenly over the 8 L2s.
__device__ __forceinline__ bool decode_work_item(const DecodeParams& p, int& split, int& kh, int& b) {
  const int i = blockIdx.x;
  const int j = i / kXcds;
  kh = j % p.num_kv_heads;
  const int u = (j / p.num_kv_heads) * kXcds + i % kXcds;
  const int units = p.batch * p.max_splits;
  if (u >= units) return false;
  split = u / p.batch;
  b = (u % p.batch + split) % p.batch;
  return true;
}

// ---------------------------------------------------------------------------
// Pass 1 tile math:
//   * S^T = K . Q^T: A = the K tile from LDS (row = key r16), B = the query
//     rows (column = query slot r16, slot s holds query s % G).  Lane l then
//     holds the scores of keys 4*(l/16)+j (j < 4) for query slot l % 16.
//   * softmax per query slot: maxima over the lane's 4 keys, then across the
//     4 lane groups (xor 16, 32).
//   * two 16-key tiles make one 32-key PV step on the matrix cores,
//     O[slot][d] += P[slot][k] V[k][d]: the lane's own probabilities of the two
//     tiles are exactly its A operand (k slots 0-3 = keys 4g..4g+3 of the even
//     tile, 4-7 = the same keys of the odd tile), and the B operand is read
//     from a row-major V tile in LDS with ds_read_b64_tr_b16, which hands lane
//     i of each 16-lane group element (i % 4) of lane 4j + i/4's 8-byte read:
//     reading V[4g + i/4][d0 + 4*(i%4)] gives lane i V[4g + j][d0 + i].
//   * 32 fp32 accumulators per lane for D = 128, whatever the group size.
// V rows in LDS are padded to D*2 + 32 bytes so the 4 rows one 16-lane group
// reads land on disjoint banks.

// Shared layout constants of pass 1.
template <int D, int G, int TILES>
struct SplitShape {
  static constexpr int KK = D / 32;
  static constexpr int CH = D / 8;
  static constexpr int RPL = 64 / CH;
  static constexpr int VL = 16 / RPL;
  static constexpr int NDT = D / 16;          // 16-column output tiles
  static constexpr int VRS = 2 * D + 32;      // padded V row in LDS (bytes)
  static constexpr int WT = 16 * TILES;
  static constexpr int KBYTES = 16 * CH * 16;                  // one K tile
  static constexpr int WAVE_BYTES = KBYTES + 32 * VRS;         // K tile + 32 V rows
  static constexpr int LOOP_BYTES = kWaves * WAVE_BYTES;
  static constexpr int EPI_BYTES = kWaves * G * D * 4 + 2 * kWaves * G * 4;
  static constexpr int SMEM = LOOP_BYTES > EPI_BYTES ? LOOP_BYTES : EPI_BYTES;
};

// The query rows of kv head kh (B operand of S^T; slot s holds query s % G).
template <int D, int G>
__device__ __forceinline__ void load_q(const DecodeParams& p, int b, int kh, uint4 (&qb)[D / 32]) {
  const int lane = threadIdx.x & 63;
  const uint16_t* qrow = static_cast<const uint16_t*>(p.q) +
                         (static_cast<int64_t>(b) * p.num_heads + kh * G + (lane & 15) % G) * D;
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk) qb[kk] = *reinterpret_cast<const uint4*>(qrow + 8 * ((lane >> 4) + 4 * kk));
}

// A 16-key tile to load ahead: kv head kh of sequence b, keys tt .. tt + 15
// (tt 16-aligned and inside the sequence).
struct NextTile {
  bool valid;
  int b, kh, tt;
};

// K/V rows of tile tt of (b, kh) into registers: lane l loads 16-byte chunk
// l % CH of rows l / CH + RPL j.
template <int D, int G, int TILES, bool kScalarBt>
__device__ __forceinline__ void load_tile_rows(const DecodeParams& p, int b, int kh, int tt,
                                               uint4 (&kr)[SplitShape<D, G, TILES>::VL],
                                               uint4 (&vr)[SplitShape<D, G, TILES>::VL]) {
  typedef SplitShape<D, G, TILES> S;
  const int lane = threadIdx.x & 63;
  const int vch = lane % S::CH;
  const int vrow = lane / S::CH;
  const int BS = p.block_size;
  const int64_t row_stride = static_cast<int64_t>(p.num_kv_heads) * D;
  const auto* bt = block_row<kScalarBt>(p, b);
  const int blk = min(max(bt[tt / BS], 0), p.num_blocks - 1);
  const int64_t row0 = static_cast<int64_t>(blk) * BS + tt % BS;
  const uint16_t* kp = static_cast<const uint16_t*>(p.k) + kh * D + (row0 + vrow) * row_stride + 8 * vch;
  const uint16_t* vp = static_cast<const uint16_t*>(p.v) + kh * D + (row0 + vrow) * row_stride + 8 * vch;
#pragma unroll
  for (int j = 0; j < S::VL; ++j) kr[j] = load_kv16(kp + S::RPL * j * row_stride);
#pragma unroll
  for (int j = 0; j < S::VL; ++j) vr[j] = load_kv16(vp + S::RPL * j * row_stride);
}

// The same as decode_wave_tiles below with the register double buffer held by
// the caller: with `preloaded` the first tile is already in buffer 0, and
// with nx.valid the last step loads tile nx into buffer 0 for the caller's
// next call (TILES is even), so a wave streams block after block without
// waiting on a fresh first load.
template <class Tag, int D, int G, int TILES, bool kScalarBt>
__device__ __forceinline__ void decode_wave_tiles_buf(const DecodeParams& p, char* smem, int b, int kh, int L,
                                                      int w0, int a, int e, const uint4 (&qb)[D / 32],
                                                      float& m_q, float& l_q, floatx4 (&acc)[D / 16],
                                                      uint4 (&kst)[2][SplitShape<D, G, TILES>::VL],
                                                      uint4 (&vst)[2][SplitShape<D, G, TILES>::VL],
                                                      bool preloaded, const NextTile& nx, int64_t slot_new) {
  typedef SplitShape<D, G, TILES> S;
  constexpr int KK = S::KK, CH = S::CH, RPL = S::RPL, VL = S::VL, NDT = S::NDT, VRS = S::VRS;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15;
  const int grp = lane >> 4;
  const int vch = lane % CH;
  const int vrow = lane / CH;
  const int BS = p.block_size;
  const int64_t row_stride = static_cast<int64_t>(p.num_kv_heads) * D;
  const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + kh * D;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + kh * D;
  const auto* bt = block_row<kScalarBt>(p, b);
  uint4* s_k = reinterpret_cast<uint4*>(smem + wave * S::WAVE_BYTES);  // [16][CH], swizzled
  char* s_v = smem + wave * S::WAVE_BYTES + S::KBYTES;                    // [32][VRS]
  {
    const int first_tile = a & ~15;
    const int last_tile = (e - 1) & ~15;
    auto load_tile = [&](int t, uint4 (&kr)[VL], uint4 (&vr)[VL]) {
      const int tt = __builtin_amdgcn_readfirstlane(min(max(w0 + 16 * t, first_tile), last_tile));
      const int blk = min(max(bt[tt / BS], 0), p.num_blocks - 1);
      const int64_t row0 = static_cast<int64_t>(blk) * BS + tt % BS;
      const uint16_t* kp = kbase + (row0 + vrow) * row_stride + 8 * vch;
      const uint16_t* vp = vbase + (row0 + vrow) * row_stride + 8 * vch;
#pragma unroll
      for (int j = 0; j < VL; ++j) kr[j] = load_kv16(kp + RPL * j * row_stride);
#pragma unroll
      for (int j = 0; j < VL; ++j) vr[j] = load_kv16(vp + RPL * j * row_stride);
    };

    // Fused append: the wave whose keys include the new token (key L - 1)
    // writes this kv head's slice of the token's K/V row to its slot and uses
    // it in place of the row it loaded from the cache.  No other workgroup
    // reads that slice, so no ordering with other workgroups is needed.
    // slot_new: the new token's slot (fused append, read by the caller), or -1.
    const int key_new = L - 1;
    const bool owns_new = slot_new >= 0 && key_new >= a && key_new < e;

    float p_even[4] = {0.f, 0.f, 0.f, 0.f};
    float alpha_even = 1.f;
    if (!preloaded) load_tile(0, kst[0], vst[0]);
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      if (t + 1 < TILES)
        load_tile(t + 1, kst[(t + 1) & 1], vst[(t + 1) & 1]);
      else if (nx.valid)
        load_tile_rows<D, G, TILES, kScalarBt>(p, nx.b, nx.kh, nx.tt, kst[(t + 1) & 1], vst[(t + 1) & 1]);
      const uint4(&kr)[VL] = kst[t & 1];
      const uint4(&vr)[VL] = vst[t & 1];
      const int tt = w0 + 16 * t;
      const bool full = tt >= a && tt + 16 <= e;

      // K tile and V rows (keys outside [a, e) zeroed) into the wave's LDS.
#pragma unroll
      for (int j = 0; j < VL; ++j) {
        const int row = vrow + RPL * j;
        s_k[row * CH + (vch ^ (row % CH))] = kr[j];
        uint4 w = vr[j];
        if (!full) {
          const int vt = tt + row;
          if (vt < a || vt >= e) w = make_uint4(0, 0, 0, 0);
        }
        *reinterpret_cast<uint4*>(s_v + ((t & 1) * 16 + row) * VRS + 16 * vch) = w;
      }
      if (owns_new && key_new >= tt && key_new < tt + 16) {
        const int row = key_new - tt;
        if (vrow == row % RPL) {
          const int64_t src = (static_cast<int64_t>(b) * p.num_kv_heads + kh) * D + 8 * vch;
          const uint4 kn = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.new_k) + src);
          const uint4 vn = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.new_v) + src);
          s_k[row * CH + (vch ^ (row % CH))] = kn;
          *reinterpret_cast<uint4*>(s_v + ((t & 1) * 16 + row) * VRS + 16 * vch) = vn;
          const int64_t dst = slot_new * row_stride + kh * D + 8 * vch;
          *reinterpret_cast<uint4*>(const_cast<uint16_t*>(static_cast<const uint16_t*>(p.k)) + dst) = kn;
          *reinterpret_cast<uint4*>(const_cast<uint16_t*>(static_cast<const uint16_t*>(p.v)) + dst) = vn;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      floatx4 sc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        sc = mfma16x16x32(Tag{}, s_k[r16 * CH + ((grp + 4 * kk) ^ (r16 % CH))], qb[kk], sc);

      float x[4];
      float mt = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = tt + 4 * grp + j;
        x[j] = (tok >= a && tok < e) ? sc[j] * p.scale_log2 : -INFINITY;
        mt = fmaxf(mt, x[j]);
      }
      mt = max_over_lane_groups(mt);
      const float mnew = fmaxf(m_q, mt);
      const float msafe = mnew == -INFINITY ? 0.f : mnew;
      const float alpha = __builtin_amdgcn_exp2f(m_q - msafe);
      float pr[4];
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pr[j] = __builtin_amdgcn_exp2f(x[j] - msafe);
        psum += pr[j];
      }
      l_q = l_q * alpha + psum;
      m_q = mnew;

      if ((t & 1) == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) p_even[j] = pr[j];
        alpha_even = alpha;
      } else {
        // One 32-key PV step.  Rescale the accumulators (rows = query slots
        // 4*grp + j, whose factors live in lanes 4*grp + j) and the even
        // tile's probabilities to the current maximum.
        const float apair = alpha_even * alpha;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float ar = __shfl(apair, 4 * grp + j);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) acc[dt][j] *= ar;
        }
        uint4 pa;
        pa.x = pack2(Tag{}, p_even[0] * alpha, p_even[1] * alpha);
        pa.y = pack2(Tag{}, p_even[2] * alpha, p_even[3] * alpha);
        pa.z = pack2(Tag{}, pr[0], pr[1]);
        pa.w = pack2(Tag{}, pr[2], pr[3]);
        const char* vrow_even = s_v + (4 * grp + r16 / 4) * VRS + 8 * (r16 % 4);
        const char* vrow_odd = vrow_even + 16 * VRS;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const uint2 lo2 = lds_read_tr16(vrow_even + 32 * dt);
          const uint2 hi2 = lds_read_tr16(vrow_odd + 32 * dt);
          acc[dt] = mfma16x16x32(Tag{}, pa, make_uint4(lo2.x, lo2.y, hi2.x, hi2.y), acc[dt]);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }

}

// One wave's pass over the TILES 16-key tiles from key w0, restricted to keys
// [a, e) (a < e): updates the running max / partial sum of query slot lane % 16
// and the PV accumulators.  L is the sequence length (the fused append owns key
// L - 1).
template <class Tag, int D, int G, int TILES>
__device__ __forceinline__ void decode_wave_tiles(const DecodeParams& p, char* smem, int b, int kh, int L,
                                                  int w0, int a, int e, const uint4 (&qb)[D / 32],
                                                  float& m_q, float& l_q, floatx4 (&acc)[D / 16]) {
  uint4 kst[2][SplitShape<D, G, TILES>::VL], vst[2][SplitShape<D, G, TILES>::VL];
  const NextTile none{false, 0, 0, 0};
  const int64_t slot_new = p.new_k != nullptr ? new_token_slot(p, b) : -1;
  decode_wave_tiles_buf<Tag, D, G, TILES, true>(p, smem, b, kh, L, w0, a, e, qb, m_q, l_q, acc, kst, vst, false, none,
                                          slot_new);
}

// Merges the 4 waves' states through LDS and writes, per query q of the group,
// either the bf16/f16 output row (direct) or the normalised partial o and its
// log2-sum-exp at partial row prow_base + q * prow_qstride.  Ends with a
// barrier, so the LDS is free again on return.
template <class Tag, int D, int G, int TILES>
__device__ __forceinline__ void decode_epilogue(const DecodeParams& p, char* smem, int b, int kh, float m_q,
                                                float l_q, const floatx4 (&acc)[D / 16], bool direct,
                                                int64_t prow_base, int64_t prow_qstride) {
  constexpr int NDT = D / 16;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15;
  const int grp = lane >> 4;
  const int qh0 = kh * G;
  // Wave totals: l summed over the 4 lane groups (every group then holds the
  // slot's total); maxima are already equal across groups.
  l_q = sum_over_lane_groups(l_q);

  __syncthreads();  // the loop's LDS is reused by the epilogue
  float* s_o = reinterpret_cast<float*>(smem);           // [kWaves][G][D]
  float* s_m = s_o + kWaves * G * D;                      // [kWaves][G]
  float* s_l = s_m + kWaves * G;                          // [kWaves][G]
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int slot = 4 * grp + j;
    if (slot < G) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) s_o[(wave * G + slot) * D + dt * 16 + r16] = acc[dt][j];
    }
  }
  if (grp == 0 && r16 < G) {
    s_m[wave * G + r16] = m_q;
    s_l[wave * G + r16] = l_q;
  }
  __syncthreads();

  uint16_t* out = static_cast<uint16_t*>(p.out) + (static_cast<int64_t>(b) * p.num_heads + qh0) * D;
  for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
    const int q = idx / D;
    const int d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w * G + q]);
    const float msafe = M == -INFINITY ? 0.f : M;
    float lsum = 0.f, osum = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = __builtin_amdgcn_exp2f(s_m[w * G + q] - msafe);
      lsum += f * s_l[w * G + q];
      osum += f * s_o[(w * G + q) * D + d];
    }
    const float o = lsum > 0.f ? osum / lsum : 0.f;
    if (direct) {
      out[idx] = pack1(Tag{}, o);
    } else {
      const int64_t prow = prow_base + static_cast<int64_t>(q) * prow_qstride;
      p.part_o[prow * D + d] = o;
      if (d == 0) p.part_lse[prow] = lsum > 0.f ? msafe + log2f(lsum) : -INFINITY;
    }
  }
  __syncthreads();
}

template <class Tag, int D, int G, int TILES>
__global__ __launch_bounds__(kThreads) void paged_decode_split(DecodeParams p) {
  static_assert(TILES % 2 == 0, "PV steps take two 16-key tiles");
  typedef SplitShape<D, G, TILES> S;
  __shared__ __align__(16) char smem[S::SMEM];

  int split, kh, b;
  if (!decode_work_item(p, split, kh, b)) return;
  const int L = seq_len(p, b);
  const int lo = p.window_left >= 0 ? max(0, L - 1 - p.window_left) : 0;
  const int s0 = split * (kWaves * S::WT);
  if (s0 >= L || s0 + kWaves * S::WT <= lo) return;

  const int wave = threadIdx.x >> 6;
  const int w0 = s0 + wave * S::WT;
  const int a = __builtin_amdgcn_readfirstlane(max(lo, w0));
  const int e = __builtin_amdgcn_readfirstlane(min(L, w0 + S::WT));

  float m_q = -INFINITY, l_q = 0.f;  // running max / this lane's partial sum, query slot lane % 16
  floatx4 acc[S::NDT];
#pragma unroll
  for (int dt = 0; dt < S::NDT; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  if (a < e) {
    uint4 qb[S::KK];
    load_q<D, G>(p, b, kh, qb);
    decode_wave_tiles<Tag, D, G, TILES>(p, smem, b, kh, L, w0, a, e, qb, m_q, l_q, acc);
  }
  const int first = lo / (kWaves * S::WT);
  const int nsplits = (L - 1) / (kWaves * S::WT) - first + 1;
  const int64_t prow0 = (static_cast<int64_t>(b) * p.num_heads + kh * G) * p.max_splits;
  decode_epilogue<Tag, D, G, TILES>(p, smem, b, kh, m_q, l_q, acc, nsplits == 1, prow0 + split, p.max_splits);
}

// ---------------------------------------------------------------------------
// Balanced pass 1 (persistent): the (sequence, kv head, key) positions are
// laid end to end -- position Hkv * cu_seqlens_k[b] + kh * L_b + j -- and
// workgroup w of W takes positions [w N / W, (w+1) N / W), N = Hkv *
// cu_seqlens_k[batch], so every workgroup streams the same number of K/V rows
// whatever the spread of lengths.  Its range is cut into segments at (b, kh)
// boundaries; per segment the 4 waves take 256-key blocks in turn (aligned to
// 16 keys, masked to the segment), and the 4 waves' states merge in LDS.  A
// segment that is a whole (b, kh) writes the output; a piece of a (b, kh) that
// crosses workgroups writes a partial to slot (w, 0) if it is the workgroup's
// first segment, else (w, 1) -- at most one of each per workgroup -- and pass 2
// combines the pieces of each (b, kh) from the owners of its first and last
// positions.
__device__ __forceinline__ int64_t owner_wg(int64_t x, int64_t n, int w) {
  return ((x + 1) * w - 1) / n;  // largest v with v * n / w <= x
}

template <class Tag, int D, int G>
__global__ __launch_bounds__(kThreads, 2) void paged_decode_persistent(DecodeParams p) {
  constexpr int TILES = 16;
  typedef SplitShape<D, G, TILES> S;
  __shared__ __align__(16) char smem[S::SMEM];
  const int W = gridDim.x;
  // Workgroup i runs on XCD i % 8: give each XCD a contiguous eighth of the
  // ranges, so the pieces of one sequence stay in one L2 (W is a multiple of 8).
  const int w = (blockIdx.x % kXcds) * (W / kXcds) + blockIdx.x / kXcds;
  const int Hkv = p.num_kv_heads;
  const int64_t N = static_cast<int64_t>(Hkv) * p.cu_seqlens_k[p.batch];
  const int64_t R0 = static_cast<int64_t>(w) * N / W;
  const int64_t R1 = static_cast<int64_t>(w + 1) * N / W;
  if (R0 >= R1) return;
  const int wave = threadIdx.x >> 6;
  int b = find_seq(p.cu_seqlens_k, p.batch, R0 / Hkv);
  int64_t x = R0;
  while (x < R1 && b < p.batch) {
    const int64_t cb = p.cu_seqlens_k[b];
    const int64_t Lraw = max(static_cast<int64_t>(p.cu_seqlens_k[b + 1]) - cb, int64_t{0});
    const int64_t base = static_cast<int64_t>(Hkv) * cb;
    if (x < base) x = base;  // only with a decreasing cu_seqlens_k
    if (x >= base + Hkv * Lraw) {
      ++b;
      continue;
    }
    const int kh = static_cast<int>((x - base) / Lraw);
    const int64_t g0 = base + kh * Lraw;
    const int64_t seg_end = min(R1, g0 + Lraw);
    const int j0 = static_cast<int>(x - g0);
    const int j1 = static_cast<int>(seg_end - g0);
    const int L = seq_len(p, b);
    const int lo = p.window_left >= 0 ? max(0, L - 1 - p.window_left) : 0;
    const int a_seg = max(j0, lo);
    const int e_seg = min(j1, L);
    float m_q = -INFINITY, l_q = 0.f;
    floatx4 acc[S::NDT];
#pragma unroll
    for (int dt = 0; dt < S::NDT; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (a_seg < e_seg) {
      uint4 qb[S::KK];
      load_q<D, G>(p, b, kh, qb);
      for (int blk0 = (a_seg & ~15) + wave * S::WT; blk0 < e_seg; blk0 += kWaves * S::WT) {
        const int a = max(a_seg, blk0);
        const int e = min(e_seg, blk0 + S::WT);
        decode_wave_tiles<Tag, D, G, TILES>(p, smem, b, kh, L, blk0, a, e, qb, m_q, l_q, acc);
      }
    }
    const bool direct = j0 == 0 && j1 == Lraw;
    const int slot = x == R0 ? 0 : 1;
    decode_epilogue<Tag, D, G, TILES>(p, smem, b, kh, m_q, l_q, acc, direct,
                                      (static_cast<int64_t>(w) * 2 + slot) * G, 1);
    x = seg_end;
  }
}

// ---------------------------------------------------------------------------
// Wave-level balanced pass 1 (stream).  A workgroup is 8 waves (one per CU):
// wave i takes kv head i % Hkv, so the Hkv waves reading one key range fetch
// the same cache rows (all heads of a key sit in one 2*Hkv*D-byte row) at the
// same time -- reading each head's range at a different time costs 5-8 % of
// the achievable HBM rate on MI355X.  The keys of the batch are laid end to
// end (key j of sequence b at cu_seqlens_k[b] + j) and cut into U = W * P
// ranges, P = 8 / Hkv; unit u = w * P + i / Hkv of workgroup w takes keys
// [u K / U, (u+1) K / U) of its head.  A wave streams its range without any
// barrier: sequence after sequence, in 256-key blocks and 32-key blocks for a
// sequence's last keys, with the register double buffer carried across blocks
// and sequences (the next block's first tile is in flight while the current
// block's last tile computes).  No workgroup turns over, no wave waits for
// another, no cross-wave merge: a sequence wholly inside the range writes its
// output from registers; a piece writes a partial to slot (u, kh, 0) (the
// range's first sequence) or (u, kh, 1) (its last), and pass 2
// (paged_decode_merge_stream) combines the pieces.
constexpr int kStreamWaves = 8;
constexpr int kStreamCuLds = 4096;

// Per-wave epilogue of a segment: query slot s < G of lane group 0 holds
// query s; acc[dt][j] of lane l is slot 4 (l / 16) + j, dim 16 dt + l % 16.
template <class Tag, int D, int G>
// whole: the segment is the sequence's whole (attended) key range; otherwise a
// piece, written to range u's slot (first ? 0 : 1).  A cascaded call writes whole
// sequences as partials too (the merge adds the shared prefix), at prefix split
// pre_splits of their rows.
__device__ __forceinline__ void decode_wave_epilogue(const DecodeParams& p, int b, int kh, float m_q, float l_q,
                                                     const floatx4 (&acc)[D / 16], bool whole, bool first,
                                                     int64_t u) {
  constexpr int NDT = D / 16;
  // The lane index passes through an empty asm statement so that the per-slot
  // addresses below are computed here, not hoisted out of the caller's loops as
  // long-lived 64-bit values (which spill at some group sizes, and the spill
  // reload's wait drains the tile loads in flight).
  int lane = threadIdx.x & 63;
  asm volatile("" : "+v"(lane));
  // One 64-bit argument carries the cascade (-1: none), so the pass holds no more
  // scalar state across its tile loop than without it.
  const bool cascade = p.whole_row0 >= 0;
  const bool direct = whole && !cascade;
  const int64_t prow_base = cascade && whole ? p.whole_row0 + static_cast<int64_t>(b) * p.num_heads + kh * G
                                             : ((u * p.num_kv_heads + kh) * 2 + (first ? 0 : 1)) * G;
  const int r16 = lane & 15;
  const int grp = lane >> 4;
  l_q = sum_over_lane_groups(l_q);
  uint16_t* out = static_cast<uint16_t*>(p.out) + (static_cast<int64_t>(b) * p.num_heads + kh * G) * D;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int slot = 4 * grp + j;
    const float l = __shfl(l_q, slot);
    const float m = __shfl(m_q, slot);
    if (slot < G) {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      if (direct) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) out[slot * D + dt * 16 + r16] = pack1(Tag{}, acc[dt][j] * inv);
      } else {
        const int64_t prow = prow_base + slot;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) p.part_o[prow * D + dt * 16 + r16] = acc[dt][j] * inv;
        if (r16 == 0) p.part_lse[prow] = l > 0.f ? m + log2f(l) : -INFINITY;
      }
    }
  }
}

template <class Tag, int D, int G, bool kDeep>
__global__ __launch_bounds__(64 * kStreamWaves, 1) void paged_decode_stream(DecodeParams p) {
  typedef SplitShape<D, G, 16> S16;
  typedef SplitShape<D, G, 2> S2;
  static_assert(S16::VL == S2::VL && S16::WAVE_BYTES == S2::WAVE_BYTES, "tile shapes shared by both block sizes");
  __shared__ __align__(16) char smem[kStreamWaves * S16::WAVE_BYTES];
  // Sequence boundaries in LDS (the host takes this path only for batches of
  // at most kStreamCuLds): every segment lookup and the binary search for a
  // range's first sequence costs LDS reads instead of dependent global loads.
  // (Read through the LDS array itself: a generic pointer would make them
  // flat loads, whose waits also drain the K/V loads in flight.)
  __shared__ uint32_t cu[kStreamCuLds + 1];
  // With a window the ranges cut the attended keys only -- [lo_b, L_b) of each
  // sequence, laid end to end, cu holding their prefix sums and win_lo the lo_b
  // -- so keys before a window start weigh nothing in the balance.
  __shared__ int win_lo[kStreamCuLds];
  // A cascaded call attends only the keys past the shared prefix here (the
  // shared count found as the prefix pass finds it): ranges over attended keys.
  const bool windowed = p.window_left >= 0 || p.shared_hint > 0;
  if (!windowed) {
    for (int i = threadIdx.x; i <= p.batch; i += 64 * kStreamWaves) cu[i] = p.cu_seqlens_k[i];
  } else {
    const int floor_keys = p.shared_hint > 0 ? find_shared_blocks<64 * kStreamWaves>(
                                                   p.cu_seqlens_k, p.block_table, p.max_blocks, p.batch,
                                                   p.block_size, p.max_seqlen_k, p.shared_hint) *
                                                   p.block_size
                                             : 0;
    attended_prefix<64 * kStreamWaves>(p, cu, win_lo, floor_keys);
  }
  __syncthreads();  // the last barrier: before any wave can leave
  // The merge's copy of the sums (after the barrier: every thread's runs are in).
  if (windowed && blockIdx.x == 0)
    for (int i = threadIdx.x; i <= p.batch; i += 64 * kStreamWaves) p.attn_cu[i] = cu[i];
  const int Hkv = p.num_kv_heads;  // divides 8 (checked on the host)
  const int P = kStreamWaves / Hkv;
  const int U = p.num_wgs;         // key ranges per head: gridDim.x * P
  const int W = gridDim.x;
  // Workgroup i runs on XCD i % 8: each XCD holds a contiguous eighth of the
  // ranges (W is a multiple of 8).  Everything below is wave-uniform.
  const int wg = (blockIdx.x % kXcds) * (W / kXcds) + blockIdx.x / kXcds;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kh = wv % Hkv;
  const int u = wg * P + wv / Hkv;
  const int64_t K = cu[p.batch];
  const int64_t R0 = static_cast<int64_t>(u) * K / U;
  const int64_t R1 = static_cast<int64_t>(u + 1) * K / U;
  if (R0 >= R1) return;  // no barrier anywhere in this kernel: waves may leave alone
  // The tile helpers use LDS area threadIdx.x / 64 of smem (8 areas here).

  // Sequence iterator over the range: keys [j0, j1) of sequence b, attended
  // keys [a, e) among them.
  struct Seg {
    bool valid;
    int b, L, j0, j1, a, e;
    bool whole;
  };
  // (With a window, positions are attended keys: offset o of sequence b is
  // key win_lo[b] + o, and every key of a segment is attended.)
  auto seg_at = [&](int64_t x, int bb) -> Seg {
    Seg g{false, 0, 0, 0, 0, 0, 0, false};
    while (x < R1 && bb < p.batch) {
      const int64_t cb = cu[bb];
      const int64_t Lraw = max(static_cast<int64_t>(cu[bb + 1]) - cb, int64_t{0});
      if (x < cb) x = cb;  // only with a decreasing cu_seqlens_k
      if (x >= R1) break;
      if (x >= cb + Lraw) {
        ++bb;
        continue;
      }
      const int o0 = static_cast<int>(x - cb);
      const int o1 = static_cast<int>(min(R1, cb + Lraw) - cb);
      if (windowed) {
        const int lo = win_lo[bb];
        const int L = lo + static_cast<int>(Lraw);
        g = Seg{true, bb, L, lo + o0, lo + o1, lo + o0, lo + o1, o0 == 0 && o1 == Lraw};
      } else {
        const int L = static_cast<int>(min(Lraw, static_cast<int64_t>(p.max_seqlen_k)));  // seq_len()
        g = Seg{true, bb, L, o0, o1, o0, min(o1, L), o0 == 0 && o1 == Lraw};
      }
      break;
    }
    return g;
  };
  uint4 kst[2][S16::VL], vst[2][S16::VL];
  Seg cur = seg_at(R0, find_seq(cu, p.batch, R0));
  bool first_seg = true;
  bool preloaded = false;
  while (cur.valid) {
    const Seg nxt = seg_at(cu[cur.b] + static_cast<int64_t>(cur.j1 - (windowed ? win_lo[cur.b] : 0)), cur.b);
    float m_q = -INFINITY, l_q = 0.f;
    floatx4 acc[S16::NDT];
#pragma unroll
    for (int dt = 0; dt < S16::NDT; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (cur.a < cur.e) {
      uint4 qb[S16::KK];
      load_q<D, G>(p, cur.b, kh, qb);
      // Fused append: only the piece holding key L - 1 needs the slot.
      const int64_t slot_new =
          p.new_k != nullptr && cur.a <= cur.L - 1 && cur.L - 1 < cur.e ? new_token_slot(p, cur.b) : -1;
      int blk0 = cur.a & ~15;
      int ntiles = ((cur.e - 1) & ~15) / 16 - blk0 / 16 + 1;
      while (ntiles > 0) {
        const bool big = ntiles >= 16;
        const int step = big ? 16 : 2;
        // The next block of the same segment is loaded behind this one; the next
        // segment's first tile is not: across the epilogue the compiler moves the
        // preloaded registers, and those moves wait for the loads anyway (measured:
        // preloading it was 0.5-1.7 % slower).
        const NextTile nt = ntiles > step ? NextTile{true, cur.b, kh, blk0 + 16 * step} : NextTile{false, 0, 0, 0};
        const int a = max(cur.a, blk0);
        const int e = min(cur.e, blk0 + 16 * step);
        if (big)
          decode_wave_tiles_buf<Tag, D, G, 16, kDeep>(p, smem, cur.b, kh, cur.L, blk0, a, e, qb, m_q, l_q, acc, kst, vst,
                                                preloaded, nt, slot_new);
        else
          decode_wave_tiles_buf<Tag, D, G, 2, kDeep>(p, smem, cur.b, kh, cur.L, blk0, a, e, qb, m_q, l_q, acc, kst, vst,
                                               preloaded, nt, slot_new);
        preloaded = nt.valid;
        blk0 += 16 * step;
        ntiles -= step;
      }
    }
    decode_wave_epilogue<Tag, D, G>(p, cur.b, kh, m_q, l_q, acc, cur.whole, first_seg, u);
    first_seg = false;
    cur = nxt;
  }
}

// Pass 2: one workgroup of 4 waves per (query head, sequence) merges the
// splits that intersect [lo, L) with log-sum-exp weights; each wave takes a
// contiguous quarter of the splits and the quarters are combined in LDS.
// Sequences with a single split were finished by pass 1 and are skipped;
// empty sequences get zeros.  A wave's log2-sum-exps and the partial rows of its
// first kChunk splits are loaded in one round (clamped indices; weights select
// the extra rows away), so the merge is two dependent rounds of loads after the
// lengths, not three.
template <class Tag, int D, int kChunk = 8>
__global__ __launch_bounds__(kThreads) void paged_decode_merge(DecodeParams p) {
  constexpr int PER = D / 64;
  __shared__ float s_o[kWaves][D];
  __shared__ float s_mw[kWaves][2];
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int L = seq_len(p, b);
  uint16_t* out = static_cast<uint16_t*>(p.out) + (static_cast<int64_t>(b) * p.num_heads + h) * D;
  if (L == 0) {
    for (int i = threadIdx.x; i < D; i += kThreads) out[i] = 0;
    // Fused append of a sequence with no keys to attend to: the first query
    // head of each kv-head group writes that head's slice of the new row.
    const int G = p.num_heads / p.num_kv_heads;
    if (p.new_k != nullptr && h % G == 0) {
      const int64_t slot = p.slot_mapping[b];
      const int kh = h / G;
      const int64_t row_stride = static_cast<int64_t>(p.num_kv_heads) * D;
      const int64_t src = (static_cast<int64_t>(b) * p.num_kv_heads + kh) * D;
      for (int i = threadIdx.x; slot >= 0 && i < D; i += kThreads) {
        const_cast<uint16_t*>(static_cast<const uint16_t*>(p.k))[slot * row_stride + kh * D + i] =
            static_cast<const uint16_t*>(p.new_k)[src + i];
        const_cast<uint16_t*>(static_cast<const uint16_t*>(p.v))[slot * row_stride + kh * D + i] =
            static_cast<const uint16_t*>(p.new_v)[src + i];
      }
    }
    return;
  }
  const int lo = p.window_left >= 0 ? max(0, L - 1 - p.window_left) : 0;
  const int first = lo / p.split_tokens;
  const int last = (L - 1) / p.split_tokens;
  if (first == last) return;
  const int n = last - first + 1;
  const int chunk = (n + kWaves - 1) / kWaves;
  const int w_first = first + wave * chunk;
  const int w_last = min(last, w_first + chunk - 1);

  const int64_t prow0 = (static_cast<int64_t>(b) * p.num_heads + h) * p.max_splits;
  const float* lse = p.part_lse + prow0;
  const int wn = w_last - w_first + 1;  // this wave's splits (none when <= 0)
  // One round: the lane's split lse and the wave's first kChunk partial rows.
  const float lse_l = lane < wn ? lse[w_first + lane] : -INFINITY;
  float pv0[kChunk][PER];
#pragma unroll
  for (int j = 0; j < kChunk; ++j) {
    const float* po = p.part_o + (prow0 + min(w_first + j, last)) * D + lane;
#pragma unroll
    for (int k = 0; k < PER; ++k) pv0[j][k] = po[64 * k];
  }
  float M = lse_l;
  for (int sp = w_first + 64 + lane; sp <= w_last; sp += 64) M = fmaxf(M, lse[sp]);  // more than 64 splits
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) M = fmaxf(M, __shfl_xor(M, m));
  const float msafe = M == -INFINITY ? 0.f : M;
  float o[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) o[i] = 0.f;
  float wsum = 0.f;
  // Groups of 64 splits: lane i owns the weight of split g + i, which every
  // lane reads with a scalar readlane; kChunk partial rows in flight at a time.
  for (int g = w_first; g <= w_last; g += 64) {
    const int cnt = min(64, w_last - g + 1);
    const float lg = g == w_first ? lse_l : (lane < cnt ? lse[g + lane] : -INFINITY);
    const float wl = lg != -INFINITY ? __builtin_amdgcn_exp2f(lg - msafe) : 0.f;
    float ws = wl;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ws += __shfl_xor(ws, m);
    wsum += ws;
    for (int i0 = 0; i0 < cnt; i0 += kChunk) {
      float wv[kChunk], pv[kChunk][PER];
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        const int i = i0 + j;
        wv[j] = i < cnt ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), i)) : 0.f;
        if (g == w_first && i0 == 0) {
#pragma unroll
          for (int k = 0; k < PER; ++k) pv[j][k] = pv0[j][k];
        } else {
          const float* po = p.part_o + (prow0 + g + min(i, cnt - 1)) * D + lane;
#pragma unroll
          for (int k = 0; k < PER; ++k) pv[j][k] = po[64 * k];
        }
      }
#pragma unroll
      for (int j = 0; j < kChunk; ++j)
#pragma unroll
        for (int k = 0; k < PER; ++k) o[k] = wv[j] != 0.f ? fmaf(wv[j], pv[j][k], o[k]) : o[k];
    }
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) s_o[wave][lane + 64 * k] = o[k];
  if (lane == 0) {
    s_mw[wave][0] = w_first <= w_last ? M : -INFINITY;
    s_mw[wave][1] = wsum;
  }
  __syncthreads();
  if (wave == 0) {
    float Mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) Mt = fmaxf(Mt, s_mw[w][0]);
    const float mt = Mt == -INFINITY ? 0.f : Mt;
    float f[kWaves], wt = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = s_mw[w][0];
      f[w] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mt);
      wt += f[w] * s_mw[w][1];
    }
    const float inv = wt > 0.f ? 1.f / wt : 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) acc = fmaf(f[w], s_o[w][lane + 64 * k], acc);
      out[lane + 64 * k] = pack1(Tag{}, acc * inv);
    }
  }
}

// Pass 2 of the persistent path: per (query head, sequence), the pieces of
// its (b, kh) from workgroups owner(g0) .. owner(g0 + L - 1), combined with
// log-sum-exp weights (a piece outside the window has weight 0).
template <class Tag, int D>
__global__ __launch_bounds__(kThreads) void paged_decode_merge_persistent(DecodeParams p) {
  constexpr int PER = D / 64;
  __shared__ float s_o[kWaves][D];
  __shared__ float s_mw[kWaves][2];
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int G = p.num_heads / p.num_kv_heads;
  const int kh = h / G;
  const int q = h % G;
  const int64_t cb = p.cu_seqlens_k[b];
  const int64_t Lraw = max(static_cast<int64_t>(p.cu_seqlens_k[b + 1]) - cb, int64_t{0});
  uint16_t* out = static_cast<uint16_t*>(p.out) + (static_cast<int64_t>(b) * p.num_heads + h) * D;
  if (Lraw == 0 || seq_len(p, b) == 0) {
    for (int i = threadIdx.x; i < D; i += kThreads) out[i] = 0;
    // Fused append of a sequence with no keys to attend to: the first query
    // head of each kv-head group writes that head's slice of the new row.
    if (p.new_k != nullptr && q == 0) {
      const int64_t slot = p.slot_mapping[b];
      const int64_t row_stride = static_cast<int64_t>(p.num_kv_heads) * D;
      const int64_t src = (static_cast<int64_t>(b) * p.num_kv_heads + kh) * D;
      for (int i = threadIdx.x; slot >= 0 && i < D; i += kThreads) {
        const_cast<uint16_t*>(static_cast<const uint16_t*>(p.k))[slot * row_stride + kh * D + i] =
            static_cast<const uint16_t*>(p.new_k)[src + i];
        const_cast<uint16_t*>(static_cast<const uint16_t*>(p.v))[slot * row_stride + kh * D + i] =
            static_cast<const uint16_t*>(p.new_v)[src + i];
      }
    }
    return;
  }
  const int W = p.num_wgs;
  const int64_t N = static_cast<int64_t>(p.num_kv_heads) * p.cu_seqlens_k[p.batch];
  const int64_t g0 = static_cast<int64_t>(p.num_kv_heads) * cb + kh * Lraw;
  if (g0 + Lraw > N) {  // inconsistent cu_seqlens_k: pass 1 did not cover these keys
    for (int i = threadIdx.x; i < D; i += kThreads) out[i] = 0;
    return;
  }
  const int64_t wa = owner_wg(g0, N, W);
  const int64_t wb = owner_wg(g0 + Lraw - 1, N, W);
  if (wa == wb) return;  // one workgroup held all of it and wrote the output
  const int s_first = wa * N / W < g0 ? 1 : 0;
  auto row = [&](int i) -> int64_t { return ((wa + i) * 2 + (i == 0 ? s_first : 0)) * G + q; };
  // With fewer positions than workgroups some own an empty range and wrote
  // nothing: their slots are skipped.
  auto piece_lse = [&](int i) -> float {
    const int64_t v = wa + i;
    return v * N / W < (v + 1) * N / W ? p.part_lse[row(i)] : -INFINITY;
  };
  const int n = static_cast<int>(wb - wa + 1);
  const int chunk = (n + kWaves - 1) / kWaves;
  const int w_first = wave * chunk;
  const int w_last = min(n - 1, w_first + chunk - 1);

  float M = -INFINITY;
  for (int i = w_first + lane; i <= w_last; i += 64) M = fmaxf(M, piece_lse(i));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) M = fmaxf(M, __shfl_xor(M, m));
  const float msafe = M == -INFINITY ? 0.f : M;
  float o[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) o[i] = 0.f;
  float wsum = 0.f;
  for (int g = w_first; g <= w_last; g += 64) {
    const int cnt = min(64, w_last - g + 1);
    const float lse = lane < cnt ? piece_lse(g + lane) : -INFINITY;
    const float wl = lane < cnt && lse != -INFINITY ? __builtin_amdgcn_exp2f(lse - msafe) : 0.f;
    float ws = wl;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ws += __shfl_xor(ws, m);
    wsum += ws;
    for (int i = 0; i < cnt; ++i) {
      const float wi =
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), i));
      if (wi == 0.f) continue;  // empty or fully windowed-out piece
      const float* po = p.part_o + row(g + i) * D + lane;
#pragma unroll
      for (int k = 0; k < PER; ++k) o[k] = fmaf(wi, po[64 * k], o[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) s_o[wave][lane + 64 * k] = o[k];
  if (lane == 0) {
    s_mw[wave][0] = w_first <= w_last ? M : -INFINITY;
    s_mw[wave][1] = wsum;
  }
  __syncthreads();
  if (wave == 0) {
    float Mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) Mt = fmaxf(Mt, s_mw[w][0]);
    const float mt = Mt == -INFINITY ? 0.f : Mt;
    float f[kWaves], wt = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = s_mw[w][0];
      f[w] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mt);
      wt += f[w] * s_mw[w][1];
    }
    const float inv = wt > 0.f ? 1.f / wt : 0.f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) acc = fmaf(f[w], s_o[w][lane + 64 * k], acc);
      out[lane + 64 * k] = pack1(Tag{}, acc * inv);
    }
  }
}

// Pass 2 of the stream path: one wave per (query head, sequence).  The pieces
// of its (b, kh) come from key ranges owner(cb) .. owner(cb + L - 1); a lane
// per piece reads its log2-sum-exp, the weights are reduced across the wave,
// and each lane then accumulates D / 64 output dims over the pieces, so the
// whole merge is three dependent rounds of loads (lengths, lse, partials).
// kChunk: pieces whose partial rows are loaded per round (16 for cascaded calls
// with more than four prefix splits, whose (sequence, head) rows gather them all).
template <class Tag, int D, int kChunk = 8>
__global__ __launch_bounds__(64) void paged_decode_merge_stream(DecodeParams p) {
  constexpr int PER = D / 64;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
  const int G = p.num_heads / p.num_kv_heads;
  const int kh = h / G;
  const int q = h % G;
  // Every length this merge needs, in one round of loads: the raw prefix sums and
  // pass 1's attended-key sums (written by pass 1 with a window; read either way,
  // used only then).  The empty asm statement makes the compiler issue all six
  // loads here, before any branch on them, so they share one memory latency
  // instead of one each.
  uint32_t c0 = p.cu_seqlens_k[b], c1 = p.cu_seqlens_k[b + 1], cn = p.cu_seqlens_k[p.batch];
  uint32_t a0 = p.attn_cu[b], a1 = p.attn_cu[b + 1], an = p.attn_cu[p.batch];
  // A cascaded call's shared count joins the same round (the item count depends on it).
  int shared = p.shared_blocks != nullptr ? *p.shared_blocks : 0;
  asm volatile("" : "+s"(c0), "+s"(c1), "+s"(cn), "+s"(a0), "+s"(a1), "+s"(an), "+s"(shared));
  const int64_t cb = c0;
  const int64_t Lraw = max(static_cast<int64_t>(c1) - cb, int64_t{0});
  const int64_t N = cn;
  uint16_t* out = static_cast<uint16_t*>(p.out) + (static_cast<int64_t>(b) * p.num_heads + h) * D;
  if (Lraw == 0 || min(Lraw, static_cast<int64_t>(p.max_seqlen_k)) == 0 || cb + Lraw > N) {
    // No keys to attend to (or an inconsistent cu_seqlens_k that pass 1 did
    // not cover): zeros; with the fused append, the first query head of each
    // kv-head group writes that head's slice of the new row.
#pragma unroll
    for (int k = 0; k < PER; ++k) out[lane + 64 * k] = 0;
    if (p.new_k != nullptr && q == 0 && Lraw == 0) {
      const int64_t slot = p.slot_mapping[b];
      if (slot >= 0) {
        const int64_t row_stride = static_cast<int64_t>(p.num_kv_heads) * D;
        const int64_t src = (static_cast<int64_t>(b) * p.num_kv_heads + kh) * D;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
          const int i = lane + 64 * k;
          const_cast<uint16_t*>(static_cast<const uint16_t*>(p.k))[slot * row_stride + kh * D + i] =
              static_cast<const uint16_t*>(p.new_k)[src + i];
          const_cast<uint16_t*>(static_cast<const uint16_t*>(p.v))[slot * row_stride + kh * D + i] =
              static_cast<const uint16_t*>(p.new_v)[src + i];
        }
      }
    }
    return;
  }
  const int U = p.num_wgs;
  // Cascaded call: the prefix pass's partial rows join pass 1's pieces.
  const bool cascade = p.shared_blocks != nullptr;
  // Pass 1's key positions: raw keys, or with a window (or a cascade) the attended
  // ones (prefix sums stored by pass 1).
  const bool attended = p.window_left >= 0 || cascade;
  const int64_t pb = attended ? static_cast<int64_t>(a0) : cb;
  const int64_t pn = attended ? static_cast<int64_t>(a1) - pb : Lraw;
  const int64_t PN = attended ? static_cast<int64_t>(an) : N;
  // Range v starts at position v PN / U; the owner of position x is the
  // largest v with v PN / U <= x.  In 32 bits whenever PN (U + 1) < 2^32 (a
  // 64-bit divide is ~10x the cost).
  const bool narrow = PN * (U + 1) < (int64_t{1} << 32);
  auto start = [&](int64_t v) -> int64_t {
    return narrow ? static_cast<int64_t>(static_cast<uint32_t>(v * PN) / static_cast<uint32_t>(U)) : v * PN / U;
  };
  auto owner = [&](int64_t x) -> int64_t {
    return narrow ? static_cast<int64_t>((static_cast<uint32_t>((x + 1) * U) - 1u) / static_cast<uint32_t>(PN))
                  : owner_wg(x, PN, U);
  };
  const int64_t wa = owner(pb);
  const int64_t wb = owner(pb + pn - 1);
  const bool whole = wa == wb;
  if (whole && !cascade) return;  // one range held all of it and wrote the output
  const int s_first = start(wa) < pb ? 1 : 0;
  // Items: pass 1's pieces (a whole sequence of a cascaded call: its one partial
  // row at prefix split pre_splits), then the prefix splits that hold shared keys.
  const int n_s = whole ? 1 : static_cast<int>(wb - wa + 1);
  const int n_p = cascade ? min(p.pre_splits, (shared * p.block_size + p.split_keys - 1) / p.split_keys) : 0;
  const int n = n_s + n_p;
  auto pre_row = [&](int sp) -> int64_t {
    return p.pre_row0 + (static_cast<int64_t>(sp) * p.batch + b) * p.num_heads + h;
  };
  auto row = [&](int i) -> int64_t {
    if (i >= n_s) return pre_row(i - n_s);
    if (whole) return pre_row(p.pre_splits);
    return (((wa + i) * p.num_kv_heads + kh) * 2 + (i == 0 ? s_first : 0)) * G + q;
  };
  // Pieces of empty ranges (fewer keys than ranges) were never written.
  auto item_valid = [&](int i) -> bool { return i >= n_s || whole || start(wa + i) < start(wa + i + 1); };
  auto piece_lse = [&](int i) -> float { return item_valid(i) ? p.part_lse[row(i)] : -INFINITY; };
  // One round of loads for the common case: lane l's piece log2-sum-exp and
  // the partial rows of the first eight pieces are issued together (clamped
  // indices, weights 0 select the extra ones away).
  const int il = min(lane, n - 1);
  const float lse0 = p.part_lse[row(il)];
  float pv0[kChunk][PER];
#pragma unroll
  for (int j = 0; j < kChunk; ++j) {
    const float* po = p.part_o + row(min(j, n - 1)) * D + lane;
#pragma unroll
    for (int k = 0; k < PER; ++k) pv0[j][k] = po[64 * k];
  }
  const float lse_l = lane < n && item_valid(lane) ? lse0 : -INFINITY;
  float M = lse_l;
  for (int i = lane + 64; i < n; i += 64) M = fmaxf(M, piece_lse(i));  // more than 64 pieces
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) M = fmaxf(M, __shfl_xor(M, m));
  const float msafe = M == -INFINITY ? 0.f : M;
  float o[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) o[k] = 0.f;
  float wsum = 0.f;
  for (int g = 0; g < n; g += 64) {
    const int cnt = min(64, n - g);
    const float lse = g == 0 ? lse_l : (lane < cnt ? piece_lse(g + lane) : -INFINITY);
    const float wl = lse != -INFINITY ? __builtin_amdgcn_exp2f(lse - msafe) : 0.f;
    float ws = wl;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ws += __shfl_xor(ws, m);
    wsum += ws;
    // Eight pieces at a time: all their loads issued before the FMAs (the
    // first eight were loaded above).  A piece with weight 0 (an empty range:
    // its row was never written, or one wholly left of the window) is
    // selected away, not multiplied.
    for (int i0 = 0; i0 < cnt; i0 += kChunk) {
      float wv[kChunk], pv[kChunk][PER];
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        const int i = i0 + j;
        wv[j] = i < cnt ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), i)) : 0.f;
        if (g == 0 && i0 == 0) {
#pragma unroll
          for (int k = 0; k < PER; ++k) pv[j][k] = pv0[j][k];
        } else {
          const float* po = p.part_o + row(g + min(i, cnt - 1)) * D + lane;
#pragma unroll
          for (int k = 0; k < PER; ++k) pv[j][k] = po[64 * k];
        }
      }
#pragma unroll
      for (int j = 0; j < kChunk; ++j)
#pragma unroll
        for (int k = 0; k < PER; ++k) o[k] = wv[j] != 0.f ? fmaf(wv[j], pv[j][k], o[k]) : o[k];
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
#pragma unroll
  for (int k = 0; k < PER; ++k) out[lane + 64 * k] = pack1(Tag{}, o[k] * inv);
}

// Zero output for a batch whose max_seqlen_k is 0 (no split workgroups run).
__global__ __launch_bounds__(256) void zero_fill_u16(uint16_t* out, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256)
    out[i] = 0;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

using oxide::device_cu_count;

// The persistent path pays off when each of its workgroups streams a long
// range: at most batch * max_seqlen_k * Hkv positions over CUs x 2 workgroups.
// Measured on MI355X: faster from ~16 k positions per workgroup (Qwen3-32B
// B=16 ctx 32k-128k: 883 vs 953 us); slower below (Qwen3-8B B=64 ctx 2k-8k,
// Qwen3-0.6B B=32 ctx 0.5k-4k), where the split grid's many short workgroups
// hide their start-up and the XCD-aware order helps more than the balance.
enum DecodePath { kPathSplit = 1, kPathPersistent = 2, kPathStream = 3, kPathRows = 4 };

// The stream pass needs the kv heads to divide its 8 waves per workgroup and
// the sequence boundaries to fit its LDS table.
bool stream_ok(int64_t batch, int64_t num_kv_heads) {
  return num_kv_heads >= 1 && num_kv_heads <= 8 && 8 % num_kv_heads == 0 && batch <= kStreamCuLds;
}

// Path by shape (measured on MI355X, K/V read rate against the 8 TB/s peak):
//   * stream when each of its key ranges holds >= ~1024 keys at the longest
//     (batch * max_seqlen_k / (CUs * 8 / Hkv)): Qwen3-8B B=64 ctx 2k-8k 74.7 %
//     (split 72.0 %), B=128 shared prefix + window 86.4 % (split 81.9 %),
//     Qwen3-32B B=16 ctx 32k-128k 79.9 % (persistent 77.7 %);
//   * below that the split grid (Qwen3-0.6B B=32 ctx 0.5k-4k: split 64 %,
//     stream 54 %: ranges of ~300 keys make the merge and the per-sequence
//     start-up dominate), and also for fewer than 16 sequences unless the
//     ranges reach 4096 keys (Qwen3-8B B=8 ctx 8k-32k: split 62 %, stream
//     60 %: each sequence in ~30 pieces; B=16 ctx 4k-16k: stream 66 %, split
//     64 %);
//   * kv head counts that do not divide 8 take the persistent pass for long
//     shapes, the split grid otherwise.
// The stream pass's keys per range if every sequence had max_seqlen_k keys.
int64_t stream_keys_per_range(int64_t batch, int64_t num_kv_heads, int64_t max_seqlen_k) {
  return batch * max_seqlen_k / (static_cast<int64_t>(device_cu_count()) * (8 / num_kv_heads));
}

// forced: the caller's choice (paged_decode_attention_path), 0 = by shape.
// rows_ok: the shape fits the row pass (oxide::rows_path_ok); callers that do not
// know the query heads pass false.
DecodePath choose_path(int64_t batch, int64_t num_kv_heads, int64_t max_seqlen_k, int forced, bool rows_ok = false) {
  if (forced == kPathRows && rows_ok) return kPathRows;
  if (forced == kPathRows) forced = kPathStream;
  if (forced == kPathStream && !stream_ok(batch, num_kv_heads)) return kPathPersistent;
  if (forced >= kPathSplit && forced <= kPathStream) return static_cast<DecodePath>(forced);
  const int64_t cus = device_cu_count();
  if (stream_ok(batch, num_kv_heads)) {
    const int64_t keys_per_range = stream_keys_per_range(batch, num_kv_heads, max_seqlen_k);
    return keys_per_range >= 1024 && (batch >= 16 || keys_per_range >= 4096) ? kPathStream : kPathSplit;
  }
  return batch * max_seqlen_k * num_kv_heads >= int64_t{16384} * 2 * cus ? kPathPersistent : kPathSplit;
}

int64_t choose_split_tokens(int64_t batch, int64_t num_kv_heads, int64_t max_seqlen_k) {
  // The longest split (fewest partials, shortest merge) that still yields at
  // least 4096 workgroups -- about eight per workgroup slot of the 256 CUs --
  // so that the ragged tail of the grid stays short.  Measured on MI355X:
  // Qwen3-8B B=64 ctx 2k-8k and Qwen3-32B B=16 ctx 32k-128k are fastest at
  // 1024, Qwen3-0.6B B=32 ctx 0.5k-4k at 256.  Grids of fewer than 2048
  // 256-key workgroups take 128-key splits: B=4 ctx 0.3k-1k 19.4 -> 16.9 us,
  // B=8 ctx 1-3000 18.4 -> 17.7 us (at 4096 workgroups, the 0.6B shape, the
  // longer merge outweighs the finer grid).
  for (int64_t st : {int64_t{1024}, int64_t{512}}) {
    if (batch * num_kv_heads * ceil_div(max_seqlen_k, st) >= 4096) return st;
  }
  return batch * num_kv_heads * ceil_div(max_seqlen_k, int64_t{256}) >= 2048 ? 256 : 128;
}

dim3 split_grid(const DecodeParams& p) {
  const int64_t units = static_cast<int64_t>(p.batch) * p.max_splits;
  return dim3(static_cast<unsigned>((units + kXcds - 1) / kXcds * kXcds * p.num_kv_heads));
}

template <class Tag, int D, int G, int TILES>
void launch_tiles(const DecodeParams& p, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((paged_decode_split<Tag, D, G, TILES>), grid, dim3(kThreads), 0, s, p);
}

template <class Tag, int D, int G>
void launch_split(const DecodeParams& p, int64_t batch, hipStream_t s) {
  (void)batch;
  const dim3 grid = split_grid(p);
  // split_tokens = kWaves * 16 * TILES.
  if (p.split_tokens == 128)
    launch_tiles<Tag, D, G, 2>(p, grid, s);
  else if (p.split_tokens == 256)
    launch_tiles<Tag, D, G, 4>(p, grid, s);
  else if (p.split_tokens == 1024)
    launch_tiles<Tag, D, G, 16>(p, grid, s);
  else
    launch_tiles<Tag, D, G, 8>(p, grid, s);
}

template <class Tag, int D>
bool dispatch_group(const DecodeParams& p, int64_t batch, int group, hipStream_t s) {
  switch (group) {
    case 1: launch_split<Tag, D, 1>(p, batch, s); return true;
    case 2: launch_split<Tag, D, 2>(p, batch, s); return true;
    case 3: launch_split<Tag, D, 3>(p, batch, s); return true;
    case 4: launch_split<Tag, D, 4>(p, batch, s); return true;
    case 5: launch_split<Tag, D, 5>(p, batch, s); return true;
    case 6: launch_split<Tag, D, 6>(p, batch, s); return true;
    case 7: launch_split<Tag, D, 7>(p, batch, s); return true;
    case 8: launch_split<Tag, D, 8>(p, batch, s); return true;
    case 16: launch_split<Tag, D, 16>(p, batch, s); return true;
    default: return false;
  }
}

// Workgroups per CU of the persistent path, at most (bounds the workspace).
constexpr int kMaxWgsPerCu = 4;
constexpr int kMaxDevices = 64;


template <class Tag, int D, int G>
void launch_persistent(DecodeParams p, hipStream_t s) {
  // One workgroup per resident slot: CUs x the kernel's occupancy.
  static std::atomic<int> occ_cache[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  int occ = occ_cache[dev % kMaxDevices].load(std::memory_order_relaxed);
  if (occ == 0) {
    oxide::RelaxedCaptureScope relaxed;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, paged_decode_persistent<Tag, D, G>, kThreads, 0) !=
        hipSuccess)
      n = 2;
    occ = std::max(1, std::min(n, 4));
    occ_cache[dev % kMaxDevices].store(occ, std::memory_order_relaxed);
  }
  p.num_wgs = device_cu_count() * occ;
  p.num_wgs -= p.num_wgs % kXcds;  // a whole number of workgroups per XCD
  hipLaunchKernelGGL((paged_decode_persistent<Tag, D, G>), dim3(static_cast<unsigned>(p.num_wgs)),
                     dim3(kThreads), 0, s, p);
  hipLaunchKernelGGL((paged_decode_merge_persistent<Tag, D>),
                     dim3(static_cast<unsigned>(p.num_heads), static_cast<unsigned>(p.batch)), dim3(kThreads),
                     0, s, p);
}

template <class Tag, int D>
bool dispatch_persistent(const DecodeParams& p, int group, hipStream_t s) {
  switch (group) {
    case 1: launch_persistent<Tag, D, 1>(p, s); return true;
    case 2: launch_persistent<Tag, D, 2>(p, s); return true;
    case 3: launch_persistent<Tag, D, 3>(p, s); return true;
    case 4: launch_persistent<Tag, D, 4>(p, s); return true;
    case 5: launch_persistent<Tag, D, 5>(p, s); return true;
    case 6: launch_persistent<Tag, D, 6>(p, s); return true;
    case 7: launch_persistent<Tag, D, 7>(p, s); return true;
    case 8: launch_persistent<Tag, D, 8>(p, s); return true;
    case 16: launch_persistent<Tag, D, 16>(p, s); return true;
    default: return false;
  }
}

template <class Tag, int D, int G>
bool launch_stream(DecodeParams p, hipStream_t s, hipEvent_t join) {
  // One workgroup of 8 waves per CU; 8 / Hkv key ranges per workgroup and head.
  int wgs = p.stream_wgs > 0 ? p.stream_wgs : device_cu_count();
  wgs -= wgs % kXcds;  // a whole number of workgroups per XCD
  p.num_wgs = wgs * (kStreamWaves / p.num_kv_heads);
  // Two tiles in flight per wave (kDeep) for ranges shorter than 1536 keys by
  // the policy's estimate.  Measured on MI355X against one tile in flight:
  // Qwen3-8B B=64 ctx 0.5k-4k 112 vs 118 us, B=16 ctx 4k-16k 125 vs 130 us
  // (estimate 1024); B=64 ctx 2k-8k 225 vs 222 us, Qwen3-32B B=16 ctx
  // 32k-128k 847 vs 832 us, B=64 ctx 2k-8k 245 vs 241 us (estimate 2047 and
  // more).  Windowed batches take it too: the shared-prefix, window-4096 batch
  // of 128 gains (266 vs 285 us; its shared blocks hit in L2) and windowed ones
  // without sharing measured even (Qwen3-8B B=64 ctx 2k-8k window 4096 170 vs
  // 171 us, B=128 ctx 4k-5k 349 vs 344 us, Qwen3-32B B=16 ctx 32k-128k window
  // 8192 110 vs 109 us).
  if (p.stream_deep)
    hipLaunchKernelGGL((paged_decode_stream<Tag, D, G, true>), dim3(static_cast<unsigned>(wgs)),
                       dim3(64 * kStreamWaves), 0, s, p);
  else
    hipLaunchKernelGGL((paged_decode_stream<Tag, D, G, false>), dim3(static_cast<unsigned>(wgs)),
                       dim3(64 * kStreamWaves), 0, s, p);
  if (join != nullptr) {
    const hipError_t e = hipStreamWaitEvent(s, join, 0);
    if (e != hipSuccess) {
      oxide::set_error(OXIDE_ERR_HIP + static_cast<int>(e));
      return true;  // the error is set; nothing more is launched
    }
  }
  // Cascaded calls with more than a few prefix splits gather more items per row.
  if (p.shared_blocks != nullptr && p.pre_splits > 4)
    hipLaunchKernelGGL((paged_decode_merge_stream<Tag, D, 16>),
                       dim3(static_cast<unsigned>(p.num_heads), static_cast<unsigned>(p.batch)), dim3(64), 0, s, p);
  else
    hipLaunchKernelGGL((paged_decode_merge_stream<Tag, D>),
                       dim3(static_cast<unsigned>(p.num_heads), static_cast<unsigned>(p.batch)), dim3(64), 0, s, p);
  return true;
}

template <class Tag, int D>
bool dispatch_stream(const DecodeParams& p, int group, hipStream_t s, hipEvent_t join) {
  switch (group) {
    case 1: return launch_stream<Tag, D, 1>(p, s, join);
    case 2: return launch_stream<Tag, D, 2>(p, s, join);
    case 3: return launch_stream<Tag, D, 3>(p, s, join);
    case 4: return launch_stream<Tag, D, 4>(p, s, join);
    case 5: return launch_stream<Tag, D, 5>(p, s, join);
    case 6: return launch_stream<Tag, D, 6>(p, s, join);
    case 7: return launch_stream<Tag, D, 7>(p, s, join);
    case 8: return launch_stream<Tag, D, 8>(p, s, join);
    case 16: return launch_stream<Tag, D, 16>(p, s, join);
    default: return false;
  }
}

// join (cascaded calls whose prefix pass runs on a side stream): an event the
// stream path's merge waits for; null otherwise.
template <class Tag>
bool dispatch(const DecodeParams& p, int64_t batch, int head_dim, int group, hipStream_t s,
              hipEvent_t join = nullptr) {
  if (p.max_splits == 0) {
    // max_seqlen_k == 0: every sequence is empty, the output is zeros.
    const int64_t n = batch * p.num_heads * head_dim;
    hipLaunchKernelGGL(zero_fill_u16, dim3(static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 4096))),
                       dim3(256), 0, s, static_cast<uint16_t*>(p.out), n);
    return true;
  }
  if (p.split_tokens == 0) {
    if (head_dim == 128) return dispatch_persistent<Tag, 128>(p, group, s);
    if (head_dim == 64) return dispatch_persistent<Tag, 64>(p, group, s);
    return false;
  }
  if (p.split_tokens == -2) {  // row pass (shape checked by the caller) + the stream merge
    DecodeParams q = p;
    oxide::launch_rows_pass1(q, std::is_same<Tag, Bf16Tag>::value, s);
    hipLaunchKernelGGL((paged_decode_merge_stream<Tag, 128>),
                       dim3(static_cast<unsigned>(q.num_heads), static_cast<unsigned>(q.batch)), dim3(64), 0, s, q);
    return true;
  }
  if (p.split_tokens < 0) {
    if (head_dim == 128) return dispatch_stream<Tag, 128>(p, group, s, join);
    if (head_dim == 64) return dispatch_stream<Tag, 64>(p, group, s, join);
    return false;
  }
  const dim3 mgrid(static_cast<unsigned>(p.num_heads), static_cast<unsigned>(batch));
  if (head_dim == 128) {
    if (!dispatch_group<Tag, 128>(p, batch, group, s)) return false;
    hipLaunchKernelGGL((paged_decode_merge<Tag, 128>), mgrid, dim3(kThreads), 0, s, p);
    return true;
  }
  if (head_dim == 64) {
    if (!dispatch_group<Tag, 64>(p, batch, group, s)) return false;
    hipLaunchKernelGGL((paged_decode_merge<Tag, 64>), mgrid, dim3(kThreads), 0, s, p);
    return true;
  }
  return false;
}

// Workspace: part_o [rows, D] f32 | part_lse [rows] f32, each 256-byte
// aligned.  Split path: a row per (sequence, query head, split); persistent
// path: two per workgroup and query of the group.
struct WorkspaceLayout {
  int64_t lse_off, total;
};
WorkspaceLayout workspace_layout(int64_t rows, int64_t head_dim) {
  WorkspaceLayout w;
  w.lse_off = ceil_div(rows * head_dim * 4, 256) * 256;
  w.total = w.lse_off + ceil_div(rows * 4, 256) * 256;
  return w;
}
int64_t split_rows(int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t max_seqlen_k) {
  return batch * num_heads * ceil_div(max_seqlen_k, choose_split_tokens(batch, num_kv_heads, max_seqlen_k));
}
// Balanced paths: two rows per range owner and query of the group; owners
// are workgroups (persistent, up to kMaxWgsPerCu per CU) or waves (stream, up
// to 2 workgroups of kWaves per CU).
int64_t persistent_rows(int64_t num_heads, int64_t num_kv_heads) {
  return 2 * static_cast<int64_t>(device_cu_count()) * std::max(kMaxWgsPerCu, 2 * kWaves) *
         (num_heads / num_kv_heads);
}

int64_t partial_rows_max(int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t max_seqlen_k) {
  return std::max({split_rows(batch, num_heads, num_kv_heads, max_seqlen_k), persistent_rows(num_heads, num_kv_heads),
                   oxide::rows_partial_rows(num_heads)});
}
// The windowed stream pass's attended-key prefix sums follow the partial rows of
// the largest layout.
int64_t attn_cu_offset(int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                       int64_t max_seqlen_k) {
  return ceil_div(workspace_layout(partial_rows_max(batch, num_heads, num_kv_heads, max_seqlen_k), head_dim).total,
                  256) * 256;
}

}  // namespace

extern "C" int64_t paged_decode_attention_path_split_tokens(int path, int64_t batch, int64_t num_kv_heads,
                                                            int64_t max_seqlen_k) {
  switch (choose_path(batch, num_kv_heads, max_seqlen_k, path >= 0 && path <= 4 ? path : 0)) {
    case kPathPersistent: return 0;
    case kPathStream: return -1;
    case kPathRows: return -2;
    default: return choose_split_tokens(batch, num_kv_heads, max_seqlen_k);
  }
}

namespace {
// Workspace of a cascaded call: the stream pass's partial rows, then the prefix
// rows ((splits + 1) per query row: the prefix splits, then the whole-sequence
// partials of the stream pass), their log2-sum-exps, the attended-key prefix
// sums, and the number of shared blocks the prefix pass found.
//
// Overlap: when the stream pass is long enough to hide it, the prefix pass runs
// beside it on a side stream (reserve CUs held back from the stream pass's grid)
// in 2048-key splits, few enough workgroups to fit those CUs two per CU.
// Otherwise the two run one after the other, the prefix pass over all CUs.
// Rates measured on MI355X (Qwen3-8B heads, 128 sequences sharing 15 blocks of
// 256 keys, window 4096): a prefix workgroup walks a 64-key tile in ~2.7 us two to
// a CU and starts in ~10 us; the stream pass reads at ~4.5 TB/s beside it.  The
// stream estimate takes every sequence at max_seqlen_k (the host knows no more),
// so ragged batches lean towards overlapping.  That batch: 272 us plain, 122 us
// one after the other, 107 us overlapped (48 CUs reserved, 64 prefix workgroups).
struct CascadeLayout {
  int64_t stream_rows, lse_off, cu_off, shared_off, total;
  int splits, split_keys;
  int reserve;  // CUs held back from the stream pass for the prefix pass; 0 = one after the other
};
constexpr int kPrefixSplitKeys = 1024;  // most keys per prefix split (a multiple of the prefill tile)
constexpr int kOverlapSplitKeys = 2048;
// Cascade modes (paged_decode_attention_shared_prefix_mode).
enum CascadeMode { kCascadeAuto = 0, kCascadeSerial = 1, kCascadeOverlap = 2, kCascadePlain = 3 };
// By shape (kCascadeAuto), the cascade runs only when the K/V bytes it saves -- the
// shared keys read once instead of once per sequence -- are worth the prefix pass's
// start-up.  Measured on MI355X (Qwen3-8B heads, page 256), plain vs cascaded:
// B=4 sharing 8192 keys 32.1 vs 53.8 us, B=8 / 4096 34.9 vs 49.4, B=16 / 2048 34.5 vs
// 45.8 (100-126 MB saved: plain wins); B=64 / 1024 129.4 vs 109.5 (264 MB), B=32 /
// 4096 103.4 vs 64.8, B=256 / 1024 197.5 vs 104.0, B=16 / 16384 176.0 vs 56.9 (cascade
// wins).  The threshold sits between: 200 MB.
bool cascade_pays(int64_t batch, int64_t num_kv_heads, int64_t head_dim, int64_t page_block_size,
                  int64_t shared_hint) {
  const double saved = static_cast<double>(batch - 1) * shared_hint * page_block_size * num_kv_heads * 4.0 * head_dim;
  return saved >= 200e6;
}
CascadeLayout cascade_layout(int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                             int64_t page_block_size, int64_t max_seqlen_k, int64_t shared_hint,
                             int mode = kCascadeAuto) {
  CascadeLayout c;
  int wgs = device_cu_count();
  wgs -= wgs % kXcds;
  c.stream_rows = 2 * static_cast<int64_t>(wgs) * (kStreamWaves / num_kv_heads) * num_heads;
  const int64_t keys = std::max<int64_t>(shared_hint, 1) * page_block_size;
  const int64_t row_tiles = ceil_div(batch * (num_heads / num_kv_heads), 128);
  const int64_t ovl_wgs = ceil_div(keys, kOverlapSplitKeys) * num_kv_heads * row_tiles;
  const int64_t reserve = ceil_div(ceil_div(ovl_wgs * 3, 4), kXcds) * kXcds;
  const double stream_us = static_cast<double>(batch) * num_kv_heads *
                           static_cast<double>(std::max<int64_t>(max_seqlen_k - keys, 0)) * 4.0 * head_dim / 4.5e6;
  const double prefix_us = 10.0 + kOverlapSplitKeys / 64 * 2.7;
  const bool overlap = mode == kCascadeOverlap || (mode == kCascadeAuto && stream_us >= prefix_us && reserve <= wgs / 4);
  if (overlap) {
    c.reserve = static_cast<int>(std::min<int64_t>(reserve, wgs / 2));
    c.split_keys = kOverlapSplitKeys;
  } else {
    // One after the other: splits of 1024 keys, halved (down to 256) while the prefix
    // pass would fill fewer workgroups than CUs: each workgroup should walk enough
    // 64-key tiles to hide its start (the shared-block scan, the queries, the first
    // tiles' latency).
    c.reserve = 0;
    c.split_keys = kPrefixSplitKeys;
    while (c.split_keys > 256 && ceil_div(keys, c.split_keys) * num_kv_heads * row_tiles < wgs) c.split_keys /= 2;
  }
  c.splits = static_cast<int>(ceil_div(keys, c.split_keys));
  const int64_t rows = c.stream_rows + (c.splits + 1) * batch * num_heads;
  const WorkspaceLayout wl = workspace_layout(rows, head_dim);
  c.lse_off = wl.lse_off;
  c.cu_off = ceil_div(wl.total, 256) * 256;
  c.shared_off = c.cu_off + ceil_div((batch + 1) * 4, 256) * 256;
  c.total = c.shared_off + 256;
  return c;
}

// The side stream of overlapped cascaded calls, one per host thread and device,
// with the two events that fork it from and join it back into the caller's stream
// (both capturable: under HIP graph capture the fork and the join become graph
// edges).  Created on the thread's first overlapped call on a device and kept
// until the process ends, at the default priority.  Per thread, so calls from
// several host threads (or graphs captured in several threads) never share one:
// each fork and join brackets that call's own work.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  bool ok = false;
};
constexpr int kMaxSideDevices = 64;
thread_local SideStream t_side[kMaxSideDevices];
SideStream* side_stream() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxSideDevices) return nullptr;
  SideStream& t = t_side[dev];
  if (!t.ok) {
    // (Re)tried on each call until it succeeds: a call that cannot create them (say,
    // under a capture mode that forbids it) runs its passes one after the other.
    oxide::RelaxedCaptureScope relaxed;
    // The events order work on this device only (the prefix pass's partials are read by
    // the merge on the same device), so they skip the system-scope fence, which makes
    // memory visible to the host and to other devices (cfg4: 108.7 -> 105.6 us).
    constexpr unsigned kFlags = hipEventDisableTiming | hipEventDisableSystemFence;
    if (!t.stream && hipStreamCreateWithFlags(&t.stream, hipStreamNonBlocking) != hipSuccess) t.stream = nullptr;
    if (!t.fork && hipEventCreateWithFlags(&t.fork, kFlags) != hipSuccess) t.fork = nullptr;
    if (!t.join && hipEventCreateWithFlags(&t.join, kFlags) != hipSuccess) t.join = nullptr;
    t.ok = t.stream && t.fork && t.join;
    if (!t.ok) (void)hipGetLastError();  // a failed creation leaves no error for the launch check
  }
  return t.ok ? &t : nullptr;
}
}  // namespace

extern "C" size_t paged_decode_attention_shared_prefix_workspace_size(int64_t batch, int64_t num_heads,
                                                                     int64_t num_kv_heads, int64_t head_dim,
                                                                     int64_t page_block_size, int64_t max_seqlen_k,
                                                                     int64_t shared_blocks_hint) {
  const size_t plain = paged_decode_attention_workspace_size(batch, num_heads, num_kv_heads, head_dim, max_seqlen_k);
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_seqlen_k <= 0 ||
      page_block_size <= 0 || shared_blocks_hint <= 0 || num_heads % num_kv_heads != 0)
    return plain;
  const int64_t hint = std::min(shared_blocks_hint, ceil_div(max_seqlen_k, page_block_size));
  const CascadeLayout c1 = cascade_layout(batch, num_heads, num_kv_heads, head_dim, page_block_size, max_seqlen_k,
                                          hint, kCascadeSerial);
  const CascadeLayout c2 = cascade_layout(batch, num_heads, num_kv_heads, head_dim, page_block_size, max_seqlen_k,
                                          hint, kCascadeOverlap);
  return std::max({plain, static_cast<size_t>(c1.total), static_cast<size_t>(c2.total)});
}

// The form paged_decode_attention_shared_prefix runs on these arguments: 1 = the
// cascade with its two passes one after the other, 2 = the cascade with the prefix
// pass beside the stream pass, 3 = the plain entries (no cascade).
extern "C" int paged_decode_attention_shared_prefix_plan(int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                                                         int64_t head_dim, int64_t page_block_size,
                                                         int64_t max_seqlen_k, int64_t shared_blocks_hint) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_seqlen_k <= 0 ||
      page_block_size <= 0 || shared_blocks_hint <= 0 || num_heads % num_kv_heads != 0)
    return kCascadePlain;
  const int64_t group = num_heads / num_kv_heads;
  if (!stream_ok(batch, num_kv_heads) || !(group <= 8 || group == 16) || (head_dim != 64 && head_dim != 128) ||
      page_block_size % 16 != 0)
    return kCascadePlain;
  const int64_t hint = std::min(shared_blocks_hint, ceil_div(max_seqlen_k, page_block_size));
  if (!cascade_pays(batch, num_kv_heads, head_dim, page_block_size, hint)) return kCascadePlain;
  const CascadeLayout c = cascade_layout(batch, num_heads, num_kv_heads, head_dim, page_block_size, max_seqlen_k, hint);
  return c.reserve > 0 ? kCascadeOverlap : kCascadeSerial;
}

extern "C" int64_t paged_decode_attention_pass1(int path, int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                                                int64_t head_dim, int64_t page_block_size, int64_t max_seqlen_k) {
  const bool rows_ok = oxide::rows_path_ok(batch, num_heads, num_kv_heads, head_dim, page_block_size);
  switch (choose_path(batch, num_kv_heads, max_seqlen_k, path >= 0 && path <= 4 ? path : 0, rows_ok)) {
    case kPathPersistent: return 0;
    case kPathStream: return -1;
    case kPathRows: return -2;
    default: return choose_split_tokens(batch, num_kv_heads, max_seqlen_k);
  }
}

extern "C" int64_t paged_decode_attention_split_tokens(int64_t batch, int64_t num_kv_heads,
                                                       int64_t max_seqlen_k) {
  return paged_decode_attention_path_split_tokens(0, batch, num_kv_heads, max_seqlen_k);
}

extern "C" size_t paged_decode_attention_workspace_size(int64_t batch, int64_t num_heads,
                                                        int64_t num_kv_heads, int64_t head_dim,
                                                        int64_t max_seqlen_k) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_seqlen_k <= 0)
    return 0;
  // Enough for every path, so a forced path (paged_decode_attention_path)
  // cannot overrun it.
  return static_cast<size_t>(attn_cu_offset(batch, num_heads, num_kv_heads, head_dim, max_seqlen_k) +
                             ceil_div((batch + 1) * 4, 256) * 256);
}

namespace {
// Shared body of the entry points; new_k / new_v / slot_mapping are null for
// plain attention; forced_path 0 = pass 1 by shape.  With compact_ws the
// workspace holds only what the chosen first pass touches (its partial rows,
// then their lse, then the attended-key prefix sums); otherwise it is laid
// out for every path and must hold paged_decode_attention_workspace_size bytes.
void decode_attention_impl(bool compact_ws, int forced_path, void* out, const void* q, const void* new_k, const void* new_v,
                           const int64_t* slot_mapping, const void* k_cache, const void* v_cache,
                           const uint32_t* cu_seqlens_k, const int32_t* block_table,
                           int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch,
                           int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                           int64_t page_block_size, int64_t max_seqlen_k, int32_t window_left,
                           float softmax_scale, void* workspace, size_t workspace_bytes, int dtype,
                           void* stream, int64_t shared_hint = 0, int cascade_mode = kCascadeAuto) {
  if (dtype != OXIDE_DTYPE_BF16 && dtype != OXIDE_DTYPE_F16) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_DTYPE);
    return;
  }
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || max_seqlen_k < 0 ||
      max_blocks_per_seq < 0 || num_blocks < 0 || num_blocks > INT32_MAX || page_block_size <= 0 || num_heads % num_kv_heads != 0) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  if (batch == 0) return;
  if (!out || !q || !cu_seqlens_k || (max_seqlen_k > 0 && (!k_cache || !v_cache || !block_table || num_blocks == 0)) ||
      !oxide::aligned16(out) || !oxide::aligned16(q) || !oxide::aligned16(k_cache) ||
      !oxide::aligned16(v_cache) || batch > 65535 || num_heads > INT32_MAX ||
      max_seqlen_k > INT32_MAX / 2 || max_blocks_per_seq * page_block_size < max_seqlen_k) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  const int64_t group = num_heads / num_kv_heads;
  if ((head_dim != 64 && head_dim != 128) || page_block_size % 16 != 0 ||
      group < 1 || (group > 8 && group != 16)) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_SHAPE);
    return;
  }
  // Never more shared blocks than the longest sequence has (the size query clamps alike).
  if (shared_hint > 0 && max_seqlen_k > 0) shared_hint = std::min(shared_hint, ceil_div(max_seqlen_k, page_block_size));
  if (shared_hint > 0 && max_seqlen_k > 0 && cascade_mode != kCascadePlain && stream_ok(batch, num_kv_heads) &&
      (group <= 8 || group == 16) &&
      (cascade_mode != kCascadeAuto || cascade_pays(batch, num_kv_heads, head_dim, page_block_size, shared_hint))) {
    // Cascaded call: the shared prefix on the matrix cores once for the whole batch,
    // the rest by the stream pass, both merged by the stream merge.
    const CascadeLayout cl = cascade_layout(batch, num_heads, num_kv_heads, head_dim, page_block_size, max_seqlen_k,
                                            shared_hint, cascade_mode);
    if (workspace_bytes < static_cast<size_t>(cl.total) || !workspace) {
      oxide::set_error(OXIDE_ERR_WORKSPACE_TOO_SMALL);
      return;
    }
    char* ws = static_cast<char*>(workspace);
    DecodeParams p{};
    p.q = q;
    p.k = k_cache;
    p.v = v_cache;
    p.cu_seqlens_k = cu_seqlens_k;
    p.block_table = block_table;
    p.part_o = reinterpret_cast<float*>(ws);
    p.part_lse = reinterpret_cast<float*>(ws + cl.lse_off);
    p.attn_cu = reinterpret_cast<uint32_t*>(ws + cl.cu_off);
    p.shared_blocks = reinterpret_cast<const int*>(ws + cl.shared_off);
    p.pre_row0 = cl.stream_rows;
    p.pre_splits = cl.splits;
    p.split_keys = cl.split_keys;
    p.whole_row0 = cl.stream_rows + static_cast<int64_t>(cl.splits) * batch * num_heads;
    p.shared_hint = static_cast<int>(shared_hint);
    p.out = out;
    p.new_k = new_k;
    p.new_v = new_v;
    p.slot_mapping = slot_mapping;
    p.max_blocks = max_blocks_per_seq;
    p.num_blocks = static_cast<int>(num_blocks);
    p.max_seqlen_k = static_cast<int>(max_seqlen_k);
    p.num_heads = static_cast<int>(num_heads);
    p.num_kv_heads = static_cast<int>(num_kv_heads);
    p.block_size = static_cast<int>(page_block_size);
    p.window_left = window_left < 0 ? -1 : window_left;
    p.split_tokens = -1;  // the stream pass
    p.stream_deep = 1;    // its ranges over the private keys are short
    p.max_splits = 1;
    p.batch = static_cast<int>(batch);
    p.scale_log2 = softmax_scale * 1.4426950408889634f;
    hipStream_t s = oxide::as_stream(stream);
    oxide::DecodePrefixArgs a{};
    a.q = q;
    a.k = k_cache;
    a.v = v_cache;
    a.cu_seqlens_k = cu_seqlens_k;
    a.block_table = block_table;
    a.max_blocks = max_blocks_per_seq;
    a.num_blocks = static_cast<int>(num_blocks);
    a.batch = static_cast<int>(batch);
    a.num_heads = static_cast<int>(num_heads);
    a.num_kv_heads = static_cast<int>(num_kv_heads);
    a.head_dim = static_cast<int>(head_dim);
    a.block_size = static_cast<int>(page_block_size);
    a.max_seqlen_k = static_cast<int>(max_seqlen_k);
    a.window_left = p.window_left;
    a.scale_log2 = p.scale_log2;
    a.part_o = p.part_o;
    a.part_lse = p.part_lse;
    a.pre_row0 = cl.stream_rows;
    a.pre_splits = cl.splits;
    a.split_keys = cl.split_keys;
    a.shared_hint = static_cast<int>(shared_hint);
    a.shared_out = reinterpret_cast<int*>(ws + cl.shared_off);
    a.bf16 = dtype == OXIDE_DTYPE_BF16;
    auto pass1_and_merge = [&](hipEvent_t join) {
      return dtype == OXIDE_DTYPE_BF16
                 ? dispatch<Bf16Tag>(p, batch, static_cast<int>(head_dim), static_cast<int>(group), s, join)
                 : dispatch<F16Tag>(p, batch, static_cast<int>(head_dim), static_cast<int>(group), s, join);
    };
    bool ok = false, overlapped = false;
    if (cl.reserve > 0) {
      // The prefix pass on the side stream, the stream pass on the caller's stream
      // over the other CUs; the merge waits for both.
      SideStream* side = side_stream();
      if (side != nullptr) {
        int wgs = device_cu_count();
        wgs -= wgs % kXcds;
        p.stream_wgs = wgs - cl.reserve;
        const hipError_t e1 = hipEventRecord(side->fork, s);
        const hipError_t e2 = e1 == hipSuccess ? hipStreamWaitEvent(side->stream, side->fork, 0) : e1;
        if (e2 != hipSuccess) {
          oxide::set_error(OXIDE_ERR_HIP + static_cast<int>(e2));
          return;
        }
        ok = oxide::launch_decode_prefix(a, side->stream);
        const hipError_t e3 = hipEventRecord(side->join, side->stream);
        if (e3 != hipSuccess) {
          oxide::set_error(OXIDE_ERR_HIP + static_cast<int>(e3));
          return;
        }
        ok = ok && pass1_and_merge(side->join);
        overlapped = true;
      }
    }
    if (!overlapped) ok = oxide::launch_decode_prefix(a, s) && pass1_and_merge(nullptr);
    if (!ok) {
      oxide::set_error(OXIDE_ERR_UNSUPPORTED_SHAPE);
      return;
    }
    oxide::check_launch();
    return;
  }
  const bool rows_ok = oxide::rows_path_ok(batch, num_heads, num_kv_heads, head_dim, page_block_size);
  const DecodePath path =
      max_seqlen_k > 0 ? choose_path(batch, num_kv_heads, max_seqlen_k, forced_path, rows_ok) : kPathSplit;
  const bool persistent = path != kPathSplit;
  const int64_t st = max_seqlen_k > 0 ? choose_split_tokens(batch, num_kv_heads, max_seqlen_k) : 1;
  const int64_t max_splits = max_seqlen_k > 0 ? ceil_div(max_seqlen_k, st) : 0;
  const WorkspaceLayout wl = workspace_layout(
      path == kPathRows ? oxide::rows_partial_rows(num_heads)
      : persistent      ? persistent_rows(num_heads, num_kv_heads)
                        : split_rows(batch, num_heads, num_kv_heads, max_seqlen_k),
      head_dim);
  const int64_t cu_off = max_seqlen_k <= 0 ? 0
                         : compact_ws ? wl.total
                                      : attn_cu_offset(batch, num_heads, num_kv_heads, head_dim, max_seqlen_k);
  const size_t need =
      max_seqlen_k <= 0 ? 0
      : compact_ws      ? static_cast<size_t>(cu_off + ceil_div((batch + 1) * 4, 256) * 256)
                        : paged_decode_attention_workspace_size(batch, num_heads, num_kv_heads, head_dim, max_seqlen_k);
  if (workspace_bytes < need || (need > 0 && !workspace)) {
    oxide::set_error(compact_ws ? OXIDE_ERR_SCRATCH_TOO_SMALL : OXIDE_ERR_WORKSPACE_TOO_SMALL);
    return;
  }
  DecodeParams p{};
  p.whole_row0 = -1;  // no cascade
  p.q = q;
  p.k = k_cache;
  p.v = v_cache;
  p.cu_seqlens_k = cu_seqlens_k;
  p.block_table = block_table;
  p.part_o = static_cast<float*>(workspace);
  p.part_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.lse_off);
  p.out = out;
  p.new_k = new_k;
  p.new_v = new_v;
  p.slot_mapping = slot_mapping;
  p.max_blocks = max_blocks_per_seq;
  p.num_blocks = static_cast<int>(num_blocks);
  p.max_seqlen_k = static_cast<int>(max_seqlen_k);
  p.num_heads = static_cast<int>(num_heads);
  p.num_kv_heads = static_cast<int>(num_kv_heads);
  p.block_size = static_cast<int>(page_block_size);
  p.window_left = window_left < 0 ? -1 : window_left;
  // 0 selects the persistent path, -1 the stream path.
  p.split_tokens = path == kPathPersistent ? 0 : path == kPathStream ? -1 : path == kPathRows ? -2 : static_cast<int>(st);
  p.stream_deep = path == kPathStream &&
                  (stream_keys_per_range(batch, num_kv_heads, max_seqlen_k) < 1536 || window_left >= 0);
  if (max_seqlen_k > 0) p.attn_cu = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + cu_off);
  p.max_splits = static_cast<int>(max_splits);
  p.batch = static_cast<int>(batch);
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  hipStream_t s = oxide::as_stream(stream);
  const bool ok = dtype == OXIDE_DTYPE_BF16
                      ? dispatch<Bf16Tag>(p, batch, static_cast<int>(head_dim), static_cast<int>(group), s)
                      : dispatch<F16Tag>(p, batch, static_cast<int>(head_dim), static_cast<int>(group), s);
  if (!ok) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_SHAPE);
    return;
  }
  oxide::check_launch();
}
}  // namespace

extern "C" void paged_decode_attention(void* out, const void* q, const void* k_cache,
                                       const void* v_cache, const uint32_t* cu_seqlens_k,
                                       const int32_t* block_table, int64_t max_blocks_per_seq,
                                       int64_t num_blocks, int64_t batch, int64_t num_heads,
                                       int64_t num_kv_heads, int64_t head_dim,
                                       int64_t page_block_size, int64_t max_seqlen_k,
                                       int32_t window_left, float softmax_scale, void* workspace,
                                       size_t workspace_bytes, int dtype, void* stream) {
  decode_attention_impl(false, 0, out, q, nullptr, nullptr, nullptr, k_cache, v_cache, cu_seqlens_k,
                        block_table, max_blocks_per_seq, num_blocks, batch, num_heads,
                        num_kv_heads, head_dim, page_block_size, max_seqlen_k, window_left,
                        softmax_scale, workspace, workspace_bytes, dtype, stream);
}

namespace {
// The fused append + attention with the pass-1 choice given (compact_ws as for
// decode_attention_impl).
void decode_append_impl(bool compact_ws, int forced_path, void* out, const void* q, const void* key, const void* value,
                        const int64_t* slot_mapping, void* k_cache, void* v_cache, const uint32_t* cu_seqlens_k,
                        const int32_t* block_table, int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch,
                        int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_block_size,
                        int64_t max_seqlen_k, int32_t window_left, float softmax_scale, void* workspace,
                        size_t workspace_bytes, int dtype, void* stream, int64_t shared_hint = 0,
                        int cascade_mode = kCascadeAuto) {
  if (batch > 0 && (!key || !value || !slot_mapping || !oxide::aligned16(key) ||
                    !oxide::aligned16(value))) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  if (max_seqlen_k <= 0) {
    // No split workgroups run: append through the plain kernel, then zeros.
    reshape_and_cache(key, value, k_cache, v_cache, slot_mapping, batch, num_kv_heads, head_dim,
                      dtype, stream);
    decode_attention_impl(compact_ws, forced_path, out, q, nullptr, nullptr, nullptr, k_cache, v_cache, cu_seqlens_k,
                          block_table, max_blocks_per_seq, num_blocks, batch, num_heads,
                          num_kv_heads, head_dim, page_block_size, max_seqlen_k, window_left,
                          softmax_scale, workspace, workspace_bytes, dtype, stream);
    return;
  }
  decode_attention_impl(compact_ws, forced_path, out, q, key, value, slot_mapping, k_cache, v_cache, cu_seqlens_k,
                        block_table, max_blocks_per_seq, num_blocks, batch, num_heads,
                        num_kv_heads, head_dim, page_block_size, max_seqlen_k, window_left,
                        softmax_scale, workspace, workspace_bytes, dtype, stream, shared_hint, cascade_mode);
}
}  // namespace

extern "C" void paged_decode_attention_append(
    void* out, const void* q, const void* key, const void* value, const int64_t* slot_mapping,
    void* k_cache, void* v_cache, const uint32_t* cu_seqlens_k, const int32_t* block_table,
    int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch, int64_t num_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t page_block_size, int64_t max_seqlen_k,
    int32_t window_left, float softmax_scale, void* workspace, size_t workspace_bytes, int dtype,
    void* stream) {
  decode_append_impl(false, 0, out, q, key, value, slot_mapping, k_cache, v_cache, cu_seqlens_k, block_table,
                     max_blocks_per_seq, num_blocks, batch, num_heads, num_kv_heads, head_dim, page_block_size,
                     max_seqlen_k, window_left, softmax_scale, workspace, workspace_bytes, dtype, stream);
}

extern "C" void paged_decode_attention_shared_prefix_mode(
    int mode, void* out, const void* q, const void* key, const void* value, const int64_t* slot_mapping,
    void* k_cache, void* v_cache, const uint32_t* cu_seqlens_k, const int32_t* block_table,
    int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch, int64_t num_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t page_block_size, int64_t max_seqlen_k, int32_t window_left, float softmax_scale,
    int64_t shared_blocks_hint, void* workspace, size_t workspace_bytes, int dtype, void* stream) {
  if (shared_blocks_hint < 0 || mode < kCascadeAuto || mode > kCascadePlain) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  if (key == nullptr && value == nullptr && slot_mapping == nullptr) {
    decode_attention_impl(false, 0, out, q, nullptr, nullptr, nullptr, k_cache, v_cache, cu_seqlens_k, block_table,
                          max_blocks_per_seq, num_blocks, batch, num_heads, num_kv_heads, head_dim, page_block_size,
                          max_seqlen_k, window_left, softmax_scale, workspace, workspace_bytes, dtype, stream,
                          shared_blocks_hint, mode);
    return;
  }
  decode_append_impl(false, 0, out, q, key, value, slot_mapping, k_cache, v_cache, cu_seqlens_k, block_table,
                     max_blocks_per_seq, num_blocks, batch, num_heads, num_kv_heads, head_dim, page_block_size,
                     max_seqlen_k, window_left, softmax_scale, workspace, workspace_bytes, dtype, stream,
                     shared_blocks_hint, mode);
}

extern "C" void paged_decode_attention_shared_prefix(
    void* out, const void* q, const void* key, const void* value, const int64_t* slot_mapping, void* k_cache,
    void* v_cache, const uint32_t* cu_seqlens_k, const int32_t* block_table, int64_t max_blocks_per_seq,
    int64_t num_blocks, int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t page_block_size, int64_t max_seqlen_k, int32_t window_left, float softmax_scale,
    int64_t shared_blocks_hint, void* workspace, size_t workspace_bytes, int dtype, void* stream) {
  paged_decode_attention_shared_prefix_mode(kCascadeAuto, out, q, key, value, slot_mapping, k_cache, v_cache,
                                            cu_seqlens_k, block_table, max_blocks_per_seq, num_blocks, batch,
                                            num_heads, num_kv_heads, head_dim, page_block_size, max_seqlen_k,
                                            window_left, softmax_scale, shared_blocks_hint, workspace,
                                            workspace_bytes, dtype, stream);
}

extern "C" void paged_decode_attention_path(
    int path, void* out, const void* q, const void* key, const void* value, const int64_t* slot_mapping,
    void* k_cache, void* v_cache, const uint32_t* cu_seqlens_k, const int32_t* block_table,
    int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch, int64_t num_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t page_block_size, int64_t max_seqlen_k,
    int32_t window_left, float softmax_scale, void* workspace, size_t workspace_bytes, int dtype,
    void* stream) {
  if (path < 0 || path > 4) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  if (key == nullptr && value == nullptr && slot_mapping == nullptr) {
    decode_attention_impl(false, path, out, q, nullptr, nullptr, nullptr, k_cache, v_cache, cu_seqlens_k, block_table,
                          max_blocks_per_seq, num_blocks, batch, num_heads, num_kv_heads, head_dim, page_block_size,
                          max_seqlen_k, window_left, softmax_scale, workspace, workspace_bytes, dtype, stream);
    return;
  }
  decode_append_impl(false, path, out, q, key, value, slot_mapping, k_cache, v_cache, cu_seqlens_k, block_table,
                     max_blocks_per_seq, num_blocks, batch, num_heads, num_kv_heads, head_dim, page_block_size,
                     max_seqlen_k, window_left, softmax_scale, workspace, workspace_bytes, dtype, stream);
}

// ---------------------------------------------------------------------------
// The same calls without a caller workspace: the partials live in a static
// device array, for callers that cannot allocate (code under graph capture,
// serving loops that forbid allocation).  Each device the library runs on
// holds its own copy of the array for the life of the process.
namespace {

constexpr size_t kScratchBytes = size_t{48} << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// `scratch` names a host-side stand-in in host code; the device address of
// each device's copy comes from hipGetSymbolAddress, taken once per device
// with that device current, and is the only form host code uses.
struct ScratchSlot {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kMaxDevices];

void* scratch_ptr() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  ScratchSlot& slot = g_scratch[dev];
  std::call_once(slot.once, [&slot] {
    oxide::RelaxedCaptureScope relaxed;  // the first call may come under graph capture
    void* ptr = nullptr;
    slot.err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (slot.err == hipSuccess) slot.ptr = ptr;
  });
  if (slot.err != hipSuccess) oxide::set_error(OXIDE_ERR_HIP + static_cast<int>(slot.err));
  return slot.ptr;
}

}  // namespace

extern "C" void paged_decode_attention_noalloc(
    void* out, const void* q, const void* key, const void* value, const int64_t* slot_mapping,
    void* k_cache, void* v_cache, const uint32_t* cu_seqlens_k, const int32_t* block_table,
    int64_t max_blocks_per_seq, int64_t num_blocks, int64_t batch, int64_t num_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t page_block_size, int64_t max_seqlen_k,
    int32_t window_left, float softmax_scale, int dtype, void* stream) {
  void* ws = scratch_ptr();
  if (ws == nullptr) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  if (key == nullptr && value == nullptr && slot_mapping == nullptr) {
    decode_attention_impl(true, 0, out, q, nullptr, nullptr, nullptr, k_cache, v_cache, cu_seqlens_k, block_table,
                          max_blocks_per_seq, num_blocks, batch, num_heads, num_kv_heads, head_dim, page_block_size,
                          max_seqlen_k, window_left, softmax_scale, ws, kScratchBytes, dtype, stream);
    return;
  }
  decode_append_impl(true, 0, out, q, key, value, slot_mapping, k_cache, v_cache, cu_seqlens_k, block_table,
                     max_blocks_per_seq, num_blocks, batch, num_heads, num_kv_heads, head_dim, page_block_size,
                     max_seqlen_k, window_left, softmax_scale, ws, kScratchBytes, dtype, stream);
}
