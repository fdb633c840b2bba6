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
// Pass 1 (paged_decode_split): one workgroup per (split, kv head, sequence).
// A split is split_tokens consecutive logical keys; its 4 waves take a quarter
// each.  A wave walks its keys in batches of NT tiles of 16 keys:
//   * K rows: lane (r16 = lane % 16, grp = lane / 16) loads 16 bytes at
//     d = 8*(grp + 4*kk) of key r16, kk < D/32: per instruction 16 rows x 64
//     contiguous bytes, the whole 256-byte row over D/32 instructions.
//   * QK^T on the matrix cores: v_mfma_f32_16x16x32_{bf16,f16} with
//     A = the G query rows of this kv head, replicated to fill the 16 MFMA
//     rows (row r holds query r % G), B = K^T (16 keys).  With the k index of
//     step kk taken as d = 8*(grp + 4*kk) + i in both operands, the dot
//     products come out in the C layout lane l -> rows 4*(l/16)+j, col l%16,
//     i.e. every lane holds the scores of key r16 for queries (4*grp+j) % G.
//     Replication means no lane needs a shuffle to find its key's scores.
//   * online softmax in the log2 domain (scale folded with log2 e), maxima
//     reduced over the 16 keys of a row with DPP, probabilities written to a
//     per-wave LDS strip [tile][key][G].
//   * PV on the VALU: V rows are loaded chunk-fixed (lane % (D/8) picks a
//     16-byte d chunk, lane / (D/8) picks the row), so each lane accumulates
//     8 d values for all G queries (8*G fp32 registers) and reads the G
//     probabilities of its row with one LDS broadcast read per row.
//   Waves are then merged through LDS and the split writes its normalised
//   partial output o (fp32, [B, Hq, max_splits, D]) and log2-sum-exp.
// Pass 2 (paged_decode_merge): one wave per (query head, sequence) merges the
// splits that intersect [lo, L) with log-sum-exp weights and writes out.
//
// Both passes read K/V exactly once; the split partials add
// 2 * Hq * (D+1) * 4 bytes per split (under 2% at split_tokens = 512).
#include <math.h>

#include <algorithm>

#include "oxide_common.hpp"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Build-time tuning knobs (defaults are the tuned values).
#ifndef OXIDE_SPLIT_TOKENS
#define OXIDE_SPLIT_TOKENS 0  // 0 = policy in choose_split_tokens
#endif
#ifndef OXIDE_DECODE_WAVES_PER_EU
#define OXIDE_DECODE_WAVES_PER_EU 0  // >0: ask the compiler for this occupancy
#endif
#if OXIDE_DECODE_WAVES_PER_EU > 0
#define OXIDE_DECODE_OCCUPANCY __attribute__((amdgpu_waves_per_eu(OXIDE_DECODE_WAVES_PER_EU)))
#else
#define OXIDE_DECODE_OCCUPANCY
#endif
#ifndef OXIDE_GRID_MODE
#define OXIDE_GRID_MODE 4  // workgroup -> (split, head, seq) order, see decode_work_item
#endif
#ifndef OXIDE_KV_NONTEMPORAL
#define OXIDE_KV_NONTEMPORAL 1  // 1 = K/V streamed with non-temporal loads
#endif

// One 16-byte K/V chunk.
__device__ __forceinline__ uint4 load_kv16(const uint16_t* p) {
#if OXIDE_KV_NONTEMPORAL
  const oxide::u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const oxide::u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
#else
  return *reinterpret_cast<const uint4*>(p);
#endif
}

struct Bf16Tag {};
struct F16Tag {};

__device__ __forceinline__ floatx4 mfma16x16x32(Bf16Tag, uint4 a, uint4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma16x16x32(F16Tag, uint4 a, uint4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Two packed 16-bit values -> fp32 (exact for both formats).
__device__ __forceinline__ void unpack2(Bf16Tag, uint32_t w, float& lo, float& hi) {
  lo = __uint_as_float(w << 16);
  hi = __uint_as_float(w & 0xffff0000u);
}
__device__ __forceinline__ void unpack2(F16Tag, uint32_t w, float& lo, float& hi) {
  const f16x2_t h = __builtin_bit_cast(f16x2_t, w);
  lo = static_cast<float>(h.x);
  hi = static_cast<float>(h.y);
}

// fp32 -> 16-bit storage, round to nearest even.
__device__ __forceinline__ uint16_t pack1(Bf16Tag, float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);  // NaN
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ uint16_t pack1(F16Tag, float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Reductions over the 16 lanes of a DPP row (lanes 16r .. 16r+15).
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror.
template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  x = fmaxf(x, dpp<0x141>(x));
  x = fmaxf(x, dpp<0x140>(x));
  return x;
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  x += dpp<0x141>(x);
  x += dpp<0x140>(x);
  return x;
}

struct DecodeParams {
  const void* q;
  const void* k;
  const void* v;
  const uint32_t* cu_seqlens_k;
  const int32_t* block_table;
  float* part_o;    // [B, Hq, max_splits, D]
  float* part_lse;  // [B, Hq, max_splits]
  void* out;        // [B, Hq, D]
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
  float scale_log2;
};

// Keys of sequence b.  Lengths beyond max_seqlen_k (a caller error) are
// clamped so that neither pass can index past the workspace or the block-table
// row; a decreasing cu_seqlens_k reads as an empty sequence.
__device__ __forceinline__ int seq_len(const DecodeParams& p, int b) {
  const int64_t n = static_cast<int64_t>(p.cu_seqlens_k[b + 1]) - p.cu_seqlens_k[b];
  return static_cast<int>(n < 0 ? 0 : (n > p.max_seqlen_k ? p.max_seqlen_k : n));
}

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kXcds = 8;  // MI355X: workgroup i runs on XCD i % 8

// Work item (split, kv head, sequence) of this workgroup; false for padding.
//   mode 0: 3-D grid (split, head, seq), seq slowest.
//   mode 1: 3-D grid (head, seq, split), split slowest.
//   mode 2/3: 1-D grid, XCD-grouped: a unit u = (seq, split) is pinned to XCD
//   u % 8 and its kv heads are consecutive workgroups there, so one XCD reads
//   all head slices of the unit's token rows together; units are numbered
//   split-major (2) or seq-major (3).
__device__ __forceinline__ bool decode_work_item(const DecodeParams& p, int& split, int& kh, int& b) {
#if OXIDE_GRID_MODE == 0
  split = blockIdx.x; kh = blockIdx.y; b = blockIdx.z;
  return true;
#elif OXIDE_GRID_MODE == 1
  kh = blockIdx.x; b = blockIdx.y; split = blockIdx.z;
  return true;
#else
  const int i = blockIdx.x;
  const int j = i / kXcds;
  kh = j % p.num_kv_heads;
  const int u = (j / p.num_kv_heads) * kXcds + i % kXcds;
  const int units = p.batch * p.max_splits;
  if (u >= units) return false;
#if OXIDE_GRID_MODE == 2
  b = u % p.batch; split = u / p.batch;
#elif OXIDE_GRID_MODE == 4
  // Split-major with the sequence rotated by the split index: unit u sits on
  // XCD u % 8, so consecutive splits of one sequence land on different XCDs
  // and ragged lengths spread evenly over the 8 L2s.
  split = u / p.batch;
  b = (u % p.batch + split) % p.batch;
#else
  split = u % p.max_splits; b = u / p.max_splits;
#endif
  return true;
#endif
}

template <class Tag, int D, int G, int TILES>
__global__ __launch_bounds__(kThreads) OXIDE_DECODE_OCCUPANCY void paged_decode_split(DecodeParams p) {
  constexpr int KK = D / 32;     // MFMA k-steps per key row
  constexpr int CH = D / 8;      // 16-byte chunks per row
  constexpr int RPL = 64 / CH;   // rows per wave-wide K/V load
  constexpr int VL = 16 / RPL;   // K (and V) loads per 16-key tile
  constexpr int GP = G < 4 ? 4 : G;  // padded LDS row (floats) for 16-byte reads
  constexpr int WT = 16 * TILES;     // keys per wave; split = kWaves * WT

  // K tile in MFMA order: row r holds 16-byte chunk c at slot c ^ (r % CH),
  // which keeps both the row-wise writes and the column-wise MFMA reads
  // spread over all LDS banks.
  __shared__ __align__(16) uint4 s_k[kWaves][16][CH];
  __shared__ __align__(16) float s_p[kWaves][16][GP];
  __shared__ __align__(16) float s_alpha[kWaves][GP];
  __shared__ __align__(16) float s_o[kWaves][G][D];
  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];

  int split, kh, b;
  if (!decode_work_item(p, split, kh, b)) return;
  const int L = seq_len(p, b);
  const int lo = p.window_left >= 0 ? max(0, L - 1 - p.window_left) : 0;
  const int s0 = split * (kWaves * WT);
  if (s0 >= L || s0 + kWaves * WT <= lo) return;  // not one of this sequence's splits

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15;
  const int grp = lane >> 4;
  const int vch = lane % CH;
  const int vrow = lane / CH;
  // This wave's keys: [a, e) inside its region [w0, w0 + WT).  Wave-uniform.
  const int w0 = s0 + wave * WT;
  const int a = __builtin_amdgcn_readfirstlane(max(lo, w0));
  const int e = __builtin_amdgcn_readfirstlane(min(L, w0 + WT));

  const int BS = p.block_size;
  const int64_t row_stride = static_cast<int64_t>(p.num_kv_heads) * D;  // elements per key row
  const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + kh * D;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + kh * D;
  const int32_t* bt = p.block_table + b * p.max_blocks;
  const int qh0 = kh * G;

  float m_run[4], l_run[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    m_run[j] = -INFINITY;
    l_run[j] = 0.f;
  }
  float acc[G][8];
#pragma unroll
  for (int q = 0; q < G; ++q)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[q][i] = 0.f;

  // Lanes that own LDS probability columns: C rows 4*grp+j with 4*grp+j < G.
  const bool writer = 4 * grp < G;

  if (a < e) {
    // A operand: query (r16 % G) of this kv head's group, chunk grp + 4*kk.
    const uint16_t* qrow = static_cast<const uint16_t*>(p.q) +
                           (static_cast<int64_t>(b) * p.num_heads + qh0 + r16 % G) * D;
    uint4 qa[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      qa[kk] = *reinterpret_cast<const uint4*>(qrow + 8 * (grp + 4 * kk));

    // Tile t covers keys [w0 + 16t, w0 + 16t + 16).  Loads are clamped to the
    // valid tiles [a & ~15, (e-1) & ~15] (a clamped tile re-reads one already
    // fetched: an L2 hit) and the compute masks keys outside [a, e), so the
    // whole walk is straight-line code: the next tile's K/V loads stay in
    // flight while the current tile computes.
    const int first_tile = a & ~15;
    const int last_tile = (e - 1) & ~15;
    uint4 kst[2][VL], vst[2][VL];
    auto load_tile = [&](int t, uint4 (&kr)[VL], uint4 (&vr)[VL]) {
      const int tt = __builtin_amdgcn_readfirstlane(min(max(w0 + 16 * t, first_tile), last_tile));
      // Block ids outside [0, num_blocks) are clamped: the output is then
      // meaningless but no access leaves the cache.
      const int blk = min(max(bt[tt / BS], 0), p.num_blocks - 1);
      const int64_t row0 = static_cast<int64_t>(blk) * BS + tt % BS;
      // K and V alike: 16 lanes cover one 256-byte head row, RPL rows per
      // instruction, the shape that streams at full HBM rate.
      const uint16_t* kp = kbase + (row0 + vrow) * row_stride + 8 * vch;
      const uint16_t* vp = vbase + (row0 + vrow) * row_stride + 8 * vch;
#pragma unroll
      for (int j = 0; j < VL; ++j) kr[j] = load_kv16(kp + RPL * j * row_stride);
#pragma unroll
      for (int j = 0; j < VL; ++j) vr[j] = load_kv16(vp + RPL * j * row_stride);
    };

    load_tile(0, kst[0], vst[0]);
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      if (t + 1 < TILES) load_tile(t + 1, kst[(t + 1) & 1], vst[(t + 1) & 1]);
      const uint4(&kr)[VL] = kst[t & 1];
      const uint4(&vr)[VL] = vst[t & 1];
      const int tt = w0 + 16 * t;

      // K tile -> LDS (row vrow + RPL*j, chunk vch), read back in the MFMA B
      // layout (key r16, chunk grp + 4*kk).  The strip is private to the wave
      // and one wave's LDS operations complete in order.
#pragma unroll
      for (int j = 0; j < VL; ++j) {
        const int row = vrow + RPL * j;
        s_k[wave][row][vch ^ (row % CH)] = kr[j];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // Scores of key tt + r16 for C rows j, in the log2 domain.
      floatx4 sc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        sc = mfma16x16x32(Tag{}, qa[kk], s_k[wave][r16][(grp + 4 * kk) ^ (r16 % CH)], sc);
      const int tok = tt + r16;
      const bool valid = tok >= a && tok < e;
      float alpha[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float x = valid ? sc[j] * p.scale_log2 : -INFINITY;
        const float mnew = fmaxf(m_run[j], row16_max(x));
        const float msafe = mnew == -INFINITY ? 0.f : mnew;
        alpha[j] = __builtin_amdgcn_exp2f(m_run[j] - msafe);
        const float pr = __builtin_amdgcn_exp2f(x - msafe);
        sc[j] = pr;
        l_run[j] = l_run[j] * alpha[j] + pr;
        m_run[j] = mnew;
      }
      if (writer) {
        if (G >= 4) {
          *reinterpret_cast<floatx4*>(&s_p[wave][r16][4 * grp]) = sc;
        } else {
#pragma unroll
          for (int j = 0; j < G; ++j) s_p[wave][r16][j] = sc[j];
        }
        if (r16 == 0) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (4 * grp + j < G) s_alpha[wave][4 * grp + j] = alpha[j];
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // PV on the VALU: this lane's V chunk (8 d values) for rows vrow + RPL*j.
#pragma unroll
      for (int q = 0; q < G; ++q) {
        const float al = s_alpha[wave][q];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[q][i] *= al;
      }
      const bool full = tt >= a && tt + 16 <= e;
#pragma unroll
      for (int j = 0; j < VL; ++j) {
        const int row = vrow + RPL * j;
        float pq[GP];
        if (G >= 4) {
#pragma unroll
          for (int q4 = 0; q4 < G; q4 += 4) {
            const floatx4 x = *reinterpret_cast<const floatx4*>(&s_p[wave][row][q4]);
            pq[q4] = x[0];
            pq[q4 + 1] = x[1];
            pq[q4 + 2] = x[2];
            pq[q4 + 3] = x[3];
          }
        } else {
#pragma unroll
          for (int q = 0; q < G; ++q) pq[q] = s_p[wave][row][q];
        }
        uint4 w = vr[j];
        if (!full) {
          // Keys outside [a, e) carry p = 0; zero their V so stale or
          // re-read cache contents (possibly NaN) cannot leak in via 0 * NaN.
          const int vt = tt + row;
          if (vt < a || vt >= e) w = make_uint4(0, 0, 0, 0);
        }
        float vf[8];
        unpack2(Tag{}, w.x, vf[0], vf[1]);
        unpack2(Tag{}, w.y, vf[2], vf[3]);
        unpack2(Tag{}, w.z, vf[4], vf[5]);
        unpack2(Tag{}, w.w, vf[6], vf[7]);
#pragma unroll
        for (int q = 0; q < G; ++q)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[q][i] = fmaf(pq[q], vf[i], acc[q][i]);
      }
      __builtin_amdgcn_wave_barrier();
    }
  }

  // Wave totals: sum l over the 16 keys of a row; sum acc over V rows.
#pragma unroll
  for (int j = 0; j < 4; ++j) l_run[j] = row16_sum(l_run[j]);
#pragma unroll
  for (int q = 0; q < G; ++q)
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int m = CH; m < 64; m <<= 1) acc[q][i] += __shfl_xor(acc[q][i], m);

  if (lane < CH) {
#pragma unroll
    for (int q = 0; q < G; ++q) {
      *reinterpret_cast<floatx4*>(&s_o[wave][q][8 * lane]) =
          floatx4{acc[q][0], acc[q][1], acc[q][2], acc[q][3]};
      *reinterpret_cast<floatx4*>(&s_o[wave][q][8 * lane + 4]) =
          floatx4{acc[q][4], acc[q][5], acc[q][6], acc[q][7]};
    }
  }
  if (writer && r16 == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (4 * grp + j < G) {
        s_m[wave][4 * grp + j] = m_run[j];
        s_l[wave][4 * grp + j] = l_run[j];
      }
    }
  }
  __syncthreads();

  // Combine the 4 waves: normalised split output o and its log2-sum-exp.
  const int first = lo / (kWaves * WT);
  const int nsplits = (L - 1) / (kWaves * WT) - first + 1;
  uint16_t* out = static_cast<uint16_t*>(p.out) + (static_cast<int64_t>(b) * p.num_heads + qh0) * D;
  const int64_t prow0 = (static_cast<int64_t>(b) * p.num_heads + qh0) * p.max_splits;
  for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
    const int q = idx / D;
    const int d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][q]);
    const float msafe = M == -INFINITY ? 0.f : M;
    float lsum = 0.f, osum = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = __builtin_amdgcn_exp2f(s_m[w][q] - msafe);
      lsum += f * s_l[w][q];
      osum += f * s_o[w][q][d];
    }
    const float o = lsum > 0.f ? osum / lsum : 0.f;
    if (nsplits == 1) {
      out[idx] = pack1(Tag{}, o);  // the only split: final output directly
    } else {
      const int64_t prow = prow0 + static_cast<int64_t>(q) * p.max_splits + split;
      p.part_o[prow * D + d] = o;
      if (d == 0) p.part_lse[prow] = lsum > 0.f ? msafe + log2f(lsum) : -INFINITY;
    }
  }
}

// Pass 2: one wave per (query head, sequence) merges the splits that
// intersect [lo, L) with log-sum-exp weights.  Sequences with a single split
// were finished by pass 1 and are skipped; empty sequences get zeros.
template <class Tag, int D>
__global__ __launch_bounds__(64) void paged_decode_merge(DecodeParams p) {
  constexpr int PER = D / 64;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
  const int L = seq_len(p, b);
  uint16_t* out = static_cast<uint16_t*>(p.out) + (static_cast<int64_t>(b) * p.num_heads + h) * D;
  if (L == 0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) out[lane + 64 * i] = 0;
    return;
  }
  const int lo = p.window_left >= 0 ? max(0, L - 1 - p.window_left) : 0;
  const int first = lo / p.split_tokens;
  const int last = (L - 1) / p.split_tokens;
  if (first == last) return;
  const int64_t prow0 = (static_cast<int64_t>(b) * p.num_heads + h) * p.max_splits;
  const float* lse = p.part_lse + prow0;
  float M = -INFINITY;
  for (int sp = first + lane; sp <= last; sp += 64) M = fmaxf(M, lse[sp]);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) M = fmaxf(M, __shfl_xor(M, m));
  const float msafe = M == -INFINITY ? 0.f : M;
  float o[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) o[i] = 0.f;
  float wsum = 0.f;
  // Splits in groups of 64: lane i owns the weight of split g + i, which every
  // lane reads with a scalar readlane while several partial rows are in flight.
  for (int g = first; g <= last; g += 64) {
    const int n = min(64, last - g + 1);
    const float wl = lane < n ? __builtin_amdgcn_exp2f(lse[g + lane] - msafe) : 0.f;
    float ws = wl;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ws += __shfl_xor(ws, m);
    wsum += ws;
    const float* po = p.part_o + (prow0 + g) * D + lane;
#pragma unroll 8
    for (int i = 0; i < n; ++i) {
      const float w =
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), i));
#pragma unroll
      for (int k = 0; k < PER; ++k) o[k] = fmaf(w, po[static_cast<int64_t>(i) * D + 64 * k], o[k]);
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) out[lane + 64 * i] = pack1(Tag{}, o[i] * inv);
}

// Zero output for a batch whose max_seqlen_k is 0 (no split workgroups run).
__global__ __launch_bounds__(256) void zero_fill_u16(uint16_t* out, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256)
    out[i] = 0;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

int64_t choose_split_tokens(int64_t batch, int64_t num_kv_heads, int64_t max_seqlen_k) {
  // 512-key splits keep the partials under 2% of the K/V bytes; fall back to
  // 256 when that would leave too few workgroups to fill 256 CUs.
  const int64_t wgs512 = batch * num_kv_heads * ceil_div(max_seqlen_k, 512);
  if (OXIDE_SPLIT_TOKENS > 0) return OXIDE_SPLIT_TOKENS;
  return wgs512 >= 4096 ? 512 : 256;
}

dim3 split_grid(const DecodeParams& p) {
#if OXIDE_GRID_MODE == 0
  return dim3(p.max_splits, p.num_kv_heads, p.batch);
#elif OXIDE_GRID_MODE == 1
  return dim3(p.num_kv_heads, p.batch, p.max_splits);
#else
  const int64_t units = static_cast<int64_t>(p.batch) * p.max_splits;
  return dim3(static_cast<unsigned>((units + kXcds - 1) / kXcds * kXcds * p.num_kv_heads));
#endif
}

template <class Tag, int D, int G>
void launch_split(const DecodeParams& p, int64_t batch, hipStream_t s) {
  const dim3 grid = split_grid(p);
  // split_tokens = kWaves * 16 * TILES.
  switch (p.split_tokens) {
    case 256: hipLaunchKernelGGL((paged_decode_split<Tag, D, G, 4>), grid, dim3(kThreads), 0, s, p); break;
#if OXIDE_SPLIT_TOKENS == 1024
    case 1024: hipLaunchKernelGGL((paged_decode_split<Tag, D, G, 16>), grid, dim3(kThreads), 0, s, p); break;
#endif
    default: hipLaunchKernelGGL((paged_decode_split<Tag, D, G, 8>), grid, dim3(kThreads), 0, s, p); break;
  }
}

template <class Tag, int D>
bool dispatch_group(const DecodeParams& p, int64_t batch, int group, hipStream_t s) {
  switch (group) {
    case 1: launch_split<Tag, D, 1>(p, batch, s); return true;
    case 2: launch_split<Tag, D, 2>(p, batch, s); return true;
    case 4: launch_split<Tag, D, 4>(p, batch, s); return true;
    case 8: launch_split<Tag, D, 8>(p, batch, s); return true;
    case 16: launch_split<Tag, D, 16>(p, batch, s); return true;
    default: return false;
  }
}

template <class Tag>
bool dispatch(const DecodeParams& p, int64_t batch, int head_dim, int group, hipStream_t s) {
  if (p.max_splits == 0) {
    // max_seqlen_k == 0: every sequence is empty, the output is zeros.
    const int64_t n = batch * p.num_heads * head_dim;
    hipLaunchKernelGGL(zero_fill_u16, dim3(static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 4096))),
                       dim3(256), 0, s, static_cast<uint16_t*>(p.out), n);
    return true;
  }
  const dim3 mgrid(static_cast<unsigned>(p.num_heads), static_cast<unsigned>(batch));
  if (head_dim == 128) {
    if (!dispatch_group<Tag, 128>(p, batch, group, s)) return false;
    hipLaunchKernelGGL((paged_decode_merge<Tag, 128>), mgrid, dim3(64), 0, s, p);
    return true;
  }
  if (head_dim == 64) {
    if (!dispatch_group<Tag, 64>(p, batch, group, s)) return false;
    hipLaunchKernelGGL((paged_decode_merge<Tag, 64>), mgrid, dim3(64), 0, s, p);
    return true;
  }
  return false;
}

// Workspace: part_o [B, Hq, splits, D] f32 | part_lse [B, Hq, splits] f32,
// each 256-byte aligned.
struct WorkspaceLayout {
  int64_t lse_off, total;
};
WorkspaceLayout workspace_layout(int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                                 int64_t head_dim, int64_t max_seqlen_k) {
  const int64_t st = choose_split_tokens(batch, num_kv_heads, max_seqlen_k);
  const int64_t rows = batch * num_heads * ceil_div(max_seqlen_k, st);
  WorkspaceLayout w;
  w.lse_off = ceil_div(rows * head_dim * 4, 256) * 256;
  w.total = w.lse_off + ceil_div(rows * 4, 256) * 256;
  return w;
}

}  // namespace

extern "C" int64_t paged_decode_attention_split_tokens(int64_t batch, int64_t num_kv_heads,
                                                       int64_t max_seqlen_k) {
  return choose_split_tokens(batch, num_kv_heads, max_seqlen_k);
}

extern "C" size_t paged_decode_attention_workspace_size(int64_t batch, int64_t num_heads,
                                                        int64_t num_kv_heads, int64_t head_dim,
                                                        int64_t max_seqlen_k) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_seqlen_k <= 0)
    return 0;
  return static_cast<size_t>(workspace_layout(batch, num_heads, num_kv_heads, head_dim, max_seqlen_k).total);
}

extern "C" void paged_decode_attention(void* out, const void* q, const void* k_cache,
                                       const void* v_cache, const uint32_t* cu_seqlens_k,
                                       const int32_t* block_table, int64_t max_blocks_per_seq,
                                       int64_t num_blocks, int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                                       int64_t head_dim, int64_t page_block_size,
                                       int64_t max_seqlen_k, int32_t window_left,
                                       float softmax_scale, void* workspace,
                                       size_t workspace_bytes, int dtype, void* stream) {
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
      (group != 1 && group != 2 && group != 4 && group != 8 && group != 16)) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_SHAPE);
    return;
  }
  const size_t need =
      paged_decode_attention_workspace_size(batch, num_heads, num_kv_heads, head_dim, max_seqlen_k);
  if (workspace_bytes < need || (need > 0 && !workspace)) {
    oxide::set_error(OXIDE_ERR_WORKSPACE_TOO_SMALL);
    return;
  }
  DecodeParams p{};
  const int64_t st = choose_split_tokens(batch, num_kv_heads, max_seqlen_k);
  const int64_t max_splits = max_seqlen_k > 0 ? ceil_div(max_seqlen_k, st) : 0;
  const WorkspaceLayout wl = workspace_layout(batch, num_heads, num_kv_heads, head_dim, max_seqlen_k);
  p.q = q;
  p.k = k_cache;
  p.v = v_cache;
  p.cu_seqlens_k = cu_seqlens_k;
  p.block_table = block_table;
  p.part_o = static_cast<float*>(workspace);
  p.part_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.lse_off);
  p.out = out;
  p.max_blocks = max_blocks_per_seq;
  p.num_blocks = static_cast<int>(num_blocks);
  p.max_seqlen_k = static_cast<int>(max_seqlen_k);
  p.num_heads = static_cast<int>(num_heads);
  p.num_kv_heads = static_cast<int>(num_kv_heads);
  p.block_size = static_cast<int>(page_block_size);
  p.window_left = window_left < 0 ? -1 : window_left;
  p.split_tokens = static_cast<int>(st);
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
