// Paged decode attention, row pass: each wave streams whole token rows (the K
// and V of all kv heads of a key, 2 KiB each at Qwen3-8B heads) instead of one
// kv head's 256-byte slices.  Same result as the other first passes of
// paged_decode.hip (the decode call of flash_attn_varlen_paged_windowed,
// crates/vllm-oxide/src/attention/flash_attn.rs:52-67, window_right = 0,
// seqlen_q = 1); its pieces are merged by paged_decode_merge_stream.
//
// Why it exists: a read-only probe of the Qwen3-8B B=64 batch read whole
// 1 KiB-per-instruction token rows ~5 % faster than per-head 256-byte slices,
// and every wave here reads two contiguous 512 KiB pages (K and V) per 256 keys.
// Measured in the full kernel on MI355X it runs at the stream pass's rate (its
// loads alone ~1 % faster, its arithmetic costs that back), so the shape policy
// never picks it; paged_decode_attention_path(4, ...) runs it on request.
//
// Work split: the batch's keys (with a window: its attended keys) are laid end to
// end and cut into one equal range per workgroup (one 8-wave workgroup per CU).  A
// workgroup walks its range sequence by sequence; inside a sequence the 2-key
// tiles go round-robin to the 8 waves, so the waves of a CU read neighbouring
// rows of the same pages at the same time.  At each sequence end the waves'
// softmax states merge through LDS (two barriers per sequence piece, none per
// tile); a whole sequence writes its output, a piece writes a partial row for the
// merge kernel at (range, kv head, 0 = the range's first sequence / 1 = its last).
//
// Lane layout (64 lanes = 4 rows of 16; row r, lane bits b3 b2 b1 b0): a tile is
// two keys.  Register R[tau][sigma] of lane (r, j) holds the 16-byte chunk
// c = 8 b1 + 4 b3 + 2 b2 + b0 (dims 8c .. 8c+7) of head r + 4 sigma of key
// tau ^ b1 of the tile.  So each load instruction reads, per row, dims 0-63 of
// one key and dims 64-127 of the other (two whole 128-byte lines), and the 16
// lanes of a row together hold every chunk of both keys of heads r and r + 4.
// The query registers are permuted the same way: Q[sigma][k] holds query
// k ^ (2 b3 + b2) of head r + 4 sigma.
//   * q.k: 16 partial dot products per lane (2 heads x 4 queries x 2 keys, 4
//     v_dot2 each), then a reduce-scatter across the 16 lanes of the row in four
//     DPP steps (row_mirror, row_half_mirror, quad_perm reversal, quad_perm xor 1)
//     instead of 16 all-reduces: the register permutations above make every step
//     but the last a plain add of a fixed register of the partner lane.  Lane
//     (r, j) ends with the score of head r + 4 b0, query 2 b3 + b2, key b1.
//   * online softmax per (head, query) in the log2 domain, one score per lane
//     (the other key's score is in lane j ^ 2), with lazy rescaling: the running
//     maximum is raised only when a tile's exceeds it by more than 2^8, so the
//     accumulators are rescaled rarely.
//   * o += p v: the two keys' probabilities are packed as a 16-bit pair and
//     broadcast within the row (DPP row_newbcast); each accumulator takes one
//     v_dot2 per tile against the V pair of its dim, repacked from the two keys'
//     registers with v_perm.
// No LDS and no matrix cores in the tile loop: the arithmetic is VALU work hidden
// behind the HBM stream.
#include <math.h>

#include "cdna4_tile.hpp"
#include "decode_common.hpp"
#include "oxide_common.hpp"

namespace {

constexpr int kRowWaves = 8;
constexpr int kRowThreads = 64 * kRowWaves;
constexpr int kRowD = 128;
constexpr int kRowHkv = 8;
constexpr int kRowG = 4;
constexpr int kRowQ = kRowHkv * kRowG;  // query heads per sequence
constexpr int kRowCuLds = 1024;         // sequences whose boundaries fit the LDS table
constexpr float kLazyGrowth = 8.f;      // log2 units the running maximum may lag

// DPP controls (gfx9 encoding).
constexpr int kDppRowMirror = 0x140;      // lane j of a row reads lane 15 - j
constexpr int kDppRowHalfMirror = 0x141;  // lane j reads (j & 8) | (7 - (j & 7))
constexpr int kDppQuadRev = 0x1B;         // quad_perm [3, 2, 1, 0]
constexpr int kDppQuadXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppRowBcast = 0x150;       // + n: row_newbcast:n (lane n of each row)

template <int kCtrl>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, true));
}
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), kCtrl, 0xf, 0xf, true));
}

__device__ __forceinline__ float dot2(Bf16Tag, uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_in_t, a), __builtin_bit_cast(bf16x2_in_t, b), c,
                                         false);
}
__device__ __forceinline__ float dot2(F16Tag, uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_in_t, a), __builtin_bit_cast(f16x2_in_t, b), c, false);
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Lane holding the probability pair of (head slot sigma, query q) after the
// reduce-scatter (its b1 = 0 lane: b0 = sigma, 2 b3 + b2 = q).
constexpr int pair_lane(int sigma, int q) { return 8 * (q >> 1) + 4 * (q & 1) + sigma; }

struct RowMergeLds {
  float o[kRowWaves][kRowQ][kRowD];
  float m[kRowWaves][kRowQ];
  float l[kRowWaves][kRowQ];
};

template <class Tag>
__global__ __launch_bounds__(kRowThreads, 1) void paged_decode_rows(DecodeParams p) {
  constexpr int D = kRowD, G = kRowG;
  __shared__ uint32_t cu[kRowCuLds + 1];
  __shared__ int win_lo[kRowCuLds];
  __shared__ __align__(16) RowMergeLds mg;
  const bool windowed = p.window_left >= 0;
  if (!windowed) {
    for (int i = threadIdx.x; i <= p.batch; i += kRowThreads) cu[i] = p.cu_seqlens_k[i];
  } else {
    attended_prefix<kRowThreads>(p, cu, win_lo);
  }
  __syncthreads();
  if (windowed && blockIdx.x == 0)
    for (int i = threadIdx.x; i <= p.batch; i += kRowThreads) p.attn_cu[i] = cu[i];
  // Workgroup i runs on XCD i % 8: each XCD holds a contiguous eighth of the
  // ranges (gridDim.x is a multiple of 8).
  const int W = gridDim.x;
  const int wg = (blockIdx.x % kXcds) * (W / kXcds) + blockIdx.x / kXcds;
  const int64_t K = cu[p.batch];
  const int64_t R0 = static_cast<int64_t>(wg) * K / W;
  const int64_t R1 = static_cast<int64_t>(wg + 1) * K / W;
  if (R0 >= R1) return;  // the whole workgroup: no barrier is left behind

  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r = lane >> 4;
  const int b0 = lane & 1, b1 = (lane >> 1) & 1, b2 = (lane >> 2) & 1, b3 = (lane >> 3) & 1;
  const int chunk = 8 * b1 + 4 * b3 + 2 * b2 + b0;
  const int qperm = 2 * b3 + b2;
  constexpr int64_t RS = static_cast<int64_t>(kRowHkv) * D;  // token row stride (elements)
  // Element offsets of the lane's chunk in a tile's first token row, for key
  // slot tau = 0 / 1 (key tau ^ b1); head slot sigma adds 4 D.
  const int64_t off0 = b1 * RS + r * D + 8 * chunk;
  const int64_t off1 = (1 - b1) * RS + r * D + 8 * chunk;
  // v_perm selectors pairing the two keys' 16-bit values of one dim (key 0 low).
  const uint32_t sel_lo = b1 ? 0x01000504u : 0x05040100u;
  const uint32_t sel_hi = b1 ? 0x03020706u : 0x07060302u;
  const int bs_shift = __builtin_ctz(static_cast<unsigned>(p.block_size));  // power of two (host-checked)
  const int bs_mask = p.block_size - 1;
  const uint16_t* kbase = static_cast<const uint16_t*>(p.k);
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v);

  struct Seg {
    bool valid;
    int b, L, a, e;
    bool whole;
  };
  // Segment of the range at position x (sequence bb or later): keys [a, e) of
  // sequence b (with a window, positions are attended keys: offset o is key
  // win_lo[b] + o).
  auto seg_at = [&](int64_t x, int bb) -> Seg {
    Seg g{false, 0, 0, 0, 0, false};
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
        g = Seg{true, bb, lo + static_cast<int>(Lraw), lo + o0, lo + o1, o0 == 0 && o1 == Lraw};
      } else {
        const int L = static_cast<int>(min(Lraw, static_cast<int64_t>(p.max_seqlen_k)));  // seq_len()
        g = Seg{true, bb, L, o0, min(o1, L), o0 == 0 && o1 == Lraw};
      }
      break;
    }
    return g;
  };

  Seg cur = seg_at(R0, find_seq(cu, p.batch, R0));
  bool first_seg = true;
  while (cur.valid) {
    const Seg nxt = seg_at(cu[cur.b] + static_cast<int64_t>(cur.e - (windowed ? win_lo[cur.b] : 0)), cur.b);
    float m = -INFINITY, l = 0.f;
    float o[2][G][8];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int q = 0; q < G; ++q)
#pragma unroll
        for (int d = 0; d < 8; ++d) o[s][q][d] = 0.f;
    const int a = cur.a, e = cur.e;
    const int ntiles = a < e ? ((e - 1) >> 1) - (a >> 1) + 1 : 0;
    const int mine = ntiles > wv ? (ntiles - 1 - wv) / kRowWaves + 1 : 0;
    if (mine > 0) {
      const int b = cur.b;
      uint4 qv[2][G];
      {
        const uint16_t* qb = static_cast<const uint16_t*>(p.q) + static_cast<int64_t>(b) * kRowQ * D + 8 * chunk;
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int k = 0; k < G; ++k)
            qv[s][k] = *reinterpret_cast<const uint4*>(qb + ((r + 4 * s) * G + (k ^ qperm)) * D);
      }
      // Fused append: the new token is key L - 1 of the segment's sequence.
      const int key_new = cur.L - 1;
      const int64_t slot_new = p.new_k != nullptr && a <= key_new && key_new < e ? new_token_slot(p, b) : -1;
      const auto* bt = block_row<true>(p, b);
      const int base = a & ~1;
      // First key of the wave's tile it (clamped to its last tile: the loads past
      // the end re-read a fetched tile and are masked, so every path through the
      // loop issues the same loads).
      auto key_of = [&](int it) { return base + 2 * (wv + kRowWaves * min(it, mine - 1)); };
      auto block_of = [&](int key0) { return min(max(bt[key0 >> bs_shift], 0), p.num_blocks - 1); };
      auto load = [&](int blk, int key0, uint4 (&kr)[2][2], uint4 (&vr)[2][2]) {
        const int64_t row0 = (static_cast<int64_t>(blk) << bs_shift) + (key0 & bs_mask);
        const uint16_t* kp = kbase + row0 * RS;
        const uint16_t* vp = vbase + row0 * RS;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          kr[0][s] = load_kv16(kp + off0 + 4 * s * D);
          kr[1][s] = load_kv16(kp + off1 + 4 * s * D);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          vr[0][s] = load_kv16(vp + off0 + 4 * s * D);
          vr[1][s] = load_kv16(vp + off1 + 4 * s * D);
        }
      };
      auto tile = [&](int key0, bool valid, uint4 (&kr)[2][2], uint4 (&vr)[2][2]) {
        const bool full = valid && key0 >= a && key0 + 2 <= e;
        if (!full) {  // keys outside [a, e): V zeroed (unused cache rows may hold NaN)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int key = key0 + (t ^ b1);
            if (!(valid && key >= a && key < e)) {
              vr[t][0] = make_uint4(0, 0, 0, 0);
              vr[t][1] = make_uint4(0, 0, 0, 0);
            }
          }
        }
        if (slot_new >= 0 && key_new >= key0 && key_new < key0 + 2) {
          // The new token's row: written to its slot and used in place of the
          // row loaded from the cache (no other workgroup reads that row).
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            if (key0 + (t ^ b1) == key_new) {
#pragma unroll
              for (int s = 0; s < 2; ++s) {
                const int64_t src = (static_cast<int64_t>(b) * kRowHkv + r + 4 * s) * D + 8 * chunk;
                const uint4 kn = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.new_k) + src);
                const uint4 vn = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.new_v) + src);
                kr[t][s] = kn;
                vr[t][s] = vn;
                const int64_t dst = slot_new * RS + (r + 4 * s) * D + 8 * chunk;
                *reinterpret_cast<uint4*>(const_cast<uint16_t*>(kbase) + dst) = kn;
                *reinterpret_cast<uint4*>(const_cast<uint16_t*>(vbase) + dst) = vn;
              }
            }
          }
        }
        // Partial q.k over the lane's 8 dims: v[sigma][k][tau].
        float v[2][G][2];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int k = 0; k < G; ++k)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
              float acc = 0.f;
#pragma unroll
              for (int i = 0; i < 4; ++i) acc = dot2(Tag{}, word(kr[t][s], i), word(qv[s][k], i), acc);
              v[s][k][t] = acc;
            }
        // Reduce-scatter over the 16 lanes of the row.
        float w[2][2][2];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int k = 0; k < 2; ++k)
#pragma unroll
            for (int t = 0; t < 2; ++t) w[s][k][t] = v[s][k][t] + dpp_f<kDppRowMirror>(v[s][k ^ 3][t ^ 1]);
        float x2[2][2];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int t = 0; t < 2; ++t) x2[s][t] = w[s][0][t] + dpp_f<kDppRowHalfMirror>(w[s][1][t ^ 1]);
        float y[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) y[s] = x2[s][0] + dpp_f<kDppQuadRev>(x2[s][1]);
        const float keep = b0 ? y[1] : y[0];
        const float send = b0 ? y[0] : y[1];
        const float sc = keep + dpp_f<kDppQuadXor1>(send);
        // This lane's score: head r + 4 b0, query qperm, key key0 + b1.
        const int key = key0 + b1;
        const float x = valid && key >= a && key < e ? sc * p.scale_log2 : -INFINITY;
        const float xm = fmaxf(x, dpp_f<kDppQuadXor2>(x));
        if (__builtin_amdgcn_ballot_w64(xm > m + kLazyGrowth) != 0) {
          const float mn = fmaxf(m, xm);
          const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
          m = mn;
          l *= alpha;
#define OXIDE_ROWS_RESCALE(S, Q)                                                   \
  {                                                                                \
    const float f = dpp_f<kDppRowBcast + pair_lane(S, Q)>(alpha);                  \
    _Pragma("unroll") for (int d = 0; d < 8; ++d) o[S][Q][d] *= f;                 \
  }
          OXIDE_ROWS_RESCALE(0, 0) OXIDE_ROWS_RESCALE(0, 1) OXIDE_ROWS_RESCALE(0, 2) OXIDE_ROWS_RESCALE(0, 3)
          OXIDE_ROWS_RESCALE(1, 0) OXIDE_ROWS_RESCALE(1, 1) OXIDE_ROWS_RESCALE(1, 2) OXIDE_ROWS_RESCALE(1, 3)
#undef OXIDE_ROWS_RESCALE
        }
        const float msafe = m == -INFINITY ? 0.f : m;
        const float pr = __builtin_amdgcn_exp2f(x - msafe);
        l += pr;
        // (p of key 0, p of key 1) as a 16-bit pair, valid in the b1 = 0 lanes.
        const uint32_t pk = pack2(Tag{}, pr, dpp_f<kDppQuadXor2>(pr));
        uint32_t vlo[2][4], vhi[2][4];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            vlo[s][i] = __builtin_amdgcn_perm(word(vr[1][s], i), word(vr[0][s], i), sel_lo);
            vhi[s][i] = __builtin_amdgcn_perm(word(vr[1][s], i), word(vr[0][s], i), sel_hi);
          }
#define OXIDE_ROWS_PV(S, Q)                                                        \
  {                                                                                \
    const uint32_t pb = dpp_u<kDppRowBcast + pair_lane(S, Q)>(pk);                 \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                \
      o[S][Q][2 * i] = dot2(Tag{}, pb, vlo[S][i], o[S][Q][2 * i]);                 \
      o[S][Q][2 * i + 1] = dot2(Tag{}, pb, vhi[S][i], o[S][Q][2 * i + 1]);         \
    }                                                                              \
  }
        OXIDE_ROWS_PV(0, 0) OXIDE_ROWS_PV(0, 1) OXIDE_ROWS_PV(0, 2) OXIDE_ROWS_PV(0, 3)
        OXIDE_ROWS_PV(1, 0) OXIDE_ROWS_PV(1, 1) OXIDE_ROWS_PV(1, 2) OXIDE_ROWS_PV(1, 3)
#undef OXIDE_ROWS_PV
      };

      uint4 ka[2][2], va[2][2], kb[2][2], vb[2][2];
      int k0 = key_of(0);
      load(block_of(k0), k0, ka, va);
      int kn1 = key_of(1);
      int blk1 = block_of(kn1);
      for (int it = 0; it < mine; it += 2) {
        load(blk1, kn1, kb, vb);
        const int kn2 = key_of(it + 2);
        const int blk2 = block_of(kn2);  // scalar load, needed only after this tile
        tile(k0, true, ka, va);
        load(blk2, kn2, ka, va);
        const int kn3 = key_of(it + 3);
        blk1 = block_of(kn3);
        tile(kn1, it + 1 < mine, kb, vb);
        k0 = kn2;
        kn1 = kn3;
      }
    }
    // Merge of the 8 waves' states of this segment through LDS.
    {
      const float lt = l + dpp_f<kDppQuadXor2>(l);
      const int hq = (r + 4 * b0) * G + qperm;
      if (b1 == 0) {
        mg.m[wv][hq] = m;
        mg.l[wv][hq] = lt;
      }
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int q = 0; q < G; ++q) {
          float4* dst = reinterpret_cast<float4*>(&mg.o[wv][(r + 4 * s) * G + q][8 * chunk]);
          dst[0] = make_float4(o[s][q][0], o[s][q][1], o[s][q][2], o[s][q][3]);
          dst[1] = make_float4(o[s][q][4], o[s][q][5], o[s][q][6], o[s][q][7]);
        }
    }
    __syncthreads();
    {
      const int row = threadIdx.x >> 4;  // query head of the sequence
      const int c = threadIdx.x & 15;    // dims 8c .. 8c+7
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kRowWaves; ++w) M = fmaxf(M, mg.m[w][row]);
      const float Ms = M == -INFINITY ? 0.f : M;
      float L = 0.f, acc[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[d] = 0.f;
#pragma unroll
      for (int w = 0; w < kRowWaves; ++w) {
        const float mw = mg.m[w][row];
        const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - Ms);
        L += f * mg.l[w][row];
        const float4 o0 = *reinterpret_cast<const float4*>(&mg.o[w][row][8 * c]);
        const float4 o1 = *reinterpret_cast<const float4*>(&mg.o[w][row][8 * c + 4]);
        acc[0] += f * o0.x, acc[1] += f * o0.y, acc[2] += f * o0.z, acc[3] += f * o0.w;
        acc[4] += f * o1.x, acc[5] += f * o1.y, acc[6] += f * o1.z, acc[7] += f * o1.w;
      }
      const float inv = L > 0.f ? 1.f / L : 0.f;
      if (cur.whole) {
        uint4 ov;
        ov.x = pack2(Tag{}, acc[0] * inv, acc[1] * inv);
        ov.y = pack2(Tag{}, acc[2] * inv, acc[3] * inv);
        ov.z = pack2(Tag{}, acc[4] * inv, acc[5] * inv);
        ov.w = pack2(Tag{}, acc[6] * inv, acc[7] * inv);
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.out) + (static_cast<int64_t>(cur.b) * kRowQ + row) * D +
                                  8 * c) = ov;
      } else {
        const int64_t prow =
            ((static_cast<int64_t>(wg) * kRowHkv + row / G) * 2 + (first_seg ? 0 : 1)) * G + row % G;
        float4* po = reinterpret_cast<float4*>(p.part_o + prow * D + 8 * c);
        po[0] = make_float4(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
        po[1] = make_float4(acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv);
        if (c == 0) p.part_lse[prow] = L > 0.f ? M + log2f(L) : -INFINITY;
      }
    }
    __syncthreads();
    first_seg = false;
    cur = nxt;
  }
}

}  // namespace

namespace oxide {

bool rows_path_ok(int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t block_size) {
  return head_dim == kRowD && num_kv_heads == kRowHkv && num_heads == kRowQ && batch >= 1 && batch <= kRowCuLds &&
         block_size >= 2 && (block_size & (block_size - 1)) == 0;
}

// Two rows (the range's first and last sequence) per key range -- one range per
// workgroup, at most one workgroup per CU -- and query head.
int64_t rows_partial_rows(int64_t num_heads) { return 2 * static_cast<int64_t>(device_cu_count()) * num_heads; }

bool launch_rows_pass1(DecodeParams& p, bool bf16, hipStream_t s) {
  int wgs = device_cu_count();
  wgs -= wgs % kXcds;  // a whole number of workgroups per XCD
  p.num_wgs = wgs;     // one key range per workgroup, for all kv heads
  if (bf16)
    hipLaunchKernelGGL(paged_decode_rows<Bf16Tag>, dim3(static_cast<unsigned>(wgs)), dim3(kRowThreads), 0, s, p);
  else
    hipLaunchKernelGGL(paged_decode_rows<F16Tag>, dim3(static_cast<unsigned>(wgs)), dim3(kRowThreads), 0, s, p);
  return true;
}

}  // namespace oxide
