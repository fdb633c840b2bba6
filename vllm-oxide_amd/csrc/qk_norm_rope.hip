// The attention prologue fused with the KV append, for gfx950: per token,
// split the merged qkv projection row, RMSNorm q and k per head, rotate them
// with RoPE at the token's position, write q for attention and k / v straight
// into their cache slots.
//
// Reference chain (Qwen3Attention::forward, crates/vllm-oxide/src/models/
// qwen3.rs:161-199): qkv.i(..) splits and reshapes, q_norm / k_norm
// (layers/rmsnorm.rs:52-87: x upcast to fp32, x / sqrt(mean(x^2) + eps),
// rounded to the dtype, times the weight, rounded), rotary_emb.forward
// (layers/rope.rs:133-163: cos / sin rows of the fp32 cache at positions[t];
// y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin in fp32, rounded to the dtype),
// then reshape_and_cache(k, v, slot_mapping).  The reference materialises q,
// k and v, the normed and the rotated copies, and reads k again for the
// append; here each input element is read once and each output written once.
//
// Rounding follows the reference step by step: products and sums are rounded
// to fp32 one at a time (no contraction into FMA), the division and the
// square root are correctly rounded.  The mean of squares is a tree sum, so it
// can differ from another backend's order in the last fp32 bit.
//
// One workgroup (256 lanes) per token.  A head is handled by 16 lanes: lane i
// holds elements [e i, e i + e) of each half (e = D / 32), i.e. the rotation
// partners x1[j] and x2[j] sit in the same lane.  16 heads per pass over the
// Hq + Hkv q and k heads; the v row is copied bitwise in 16-byte pieces.
#include <math.h>

#include "cdna4_tile.hpp"
#include "oxide_common.hpp"

namespace {

constexpr int kRopeThreads = 256;
constexpr int kLanesPerHead = 16;

__device__ __forceinline__ float to_f32(Bf16Tag, uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }
__device__ __forceinline__ float to_f32(F16Tag, uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
template <class Tag>
__device__ __forceinline__ float round_to(float x) {
  return to_f32(Tag{}, pack1(Tag{}, x));
}

struct RopeParams {
  uint16_t* q_out;            // [T, Hq, D]
  uint16_t* k_out;            // [T, Hkv, D] or null
  const uint16_t* qkv;        // [T, qkv_stride], row = q | k | v
  const uint16_t* q_weight;   // [D] or null (no norm)
  const uint16_t* k_weight;   // [D] or null
  const float* cos_sin;       // [max_position, D]
  const int32_t* positions;   // [T]
  uint16_t* key_cache;        // [slots, Hkv, D]
  uint16_t* value_cache;
  const int64_t* slot_mapping;  // [T], -1 = skip
  int64_t qkv_stride;
  int max_position;
  int num_heads;
  int num_kv_heads;
  float eps;
  bool vec_v;  // v row and cache rows 16-byte aligned
};

template <class Tag, int D>
__global__ __launch_bounds__(kRopeThreads) void qk_norm_rope_cache_kernel(RopeParams p) {
  // Every product and sum is rounded on its own, as in the reference.
#pragma clang fp contract(off)
  constexpr int E = D / 2 / kLanesPerHead;  // elements per lane per half
  const int64_t t = blockIdx.x;
  const int sub = threadIdx.x % kLanesPerHead;
  const int slot_in_pass = threadIdx.x / kLanesPerHead;
  int pos = p.positions[t];
  pos = min(max(pos, 0), p.max_position - 1);
  const float* cs = p.cos_sin + static_cast<int64_t>(pos) * D;
  const uint16_t* row = p.qkv + t * p.qkv_stride;
  const int64_t slot = p.slot_mapping ? p.slot_mapping[t] : -1;
  const int heads = p.num_heads + p.num_kv_heads;

  float c[E], s[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    c[e] = cs[sub * E + e];
    s[e] = cs[D / 2 + sub * E + e];
  }

  for (int h = slot_in_pass; h < heads; h += kRopeThreads / kLanesPerHead) {
    const bool is_q = h < p.num_heads;
    const uint16_t* src = row + static_cast<int64_t>(h) * D;
    float x1[E], x2[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      x1[e] = to_f32(Tag{}, src[sub * E + e]);
      x2[e] = to_f32(Tag{}, src[D / 2 + sub * E + e]);
    }
    const uint16_t* w = is_q ? p.q_weight : p.k_weight;
    if (w != nullptr) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) ss = ss + (x1[e] * x1[e] + x2[e] * x2[e]);
#pragma unroll
      for (int m = 1; m < kLanesPerHead; m <<= 1) ss = ss + __shfl_xor(ss, m);
      const float sd = sqrtf(ss / static_cast<float>(D) + p.eps);  // correctly rounded / and sqrt
#pragma unroll
      for (int e = 0; e < E; ++e) {
        x1[e] = round_to<Tag>(round_to<Tag>(x1[e] / sd) * to_f32(Tag{}, w[sub * E + e]));
        x2[e] = round_to<Tag>(round_to<Tag>(x2[e] / sd) * to_f32(Tag{}, w[D / 2 + sub * E + e]));
      }
    }
    uint16_t y1[E], y2[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      y1[e] = pack1(Tag{}, x1[e] * c[e] - x2[e] * s[e]);
      y2[e] = pack1(Tag{}, x2[e] * c[e] + x1[e] * s[e]);
    }
    uint16_t* dst0;
    uint16_t* dst1 = nullptr;
    if (is_q) {
      dst0 = p.q_out + (t * p.num_heads + h) * D;
    } else {
      const int kh = h - p.num_heads;
      dst0 = p.k_out ? p.k_out + (t * p.num_kv_heads + kh) * D : nullptr;
      dst1 = slot >= 0 ? p.key_cache + (slot * p.num_kv_heads + kh) * D : nullptr;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (dst0) {
        dst0[sub * E + e] = y1[e];
        dst0[D / 2 + sub * E + e] = y2[e];
      }
      if (dst1) {
        dst1[sub * E + e] = y1[e];
        dst1[D / 2 + sub * E + e] = y2[e];
      }
    }
  }

  // v: bitwise copy of the row's last Hkv * D elements into the slot.
  if (slot >= 0) {
    const uint16_t* vsrc = row + static_cast<int64_t>(heads) * D;
    uint16_t* vdst = p.value_cache + slot * p.num_kv_heads * D;
    const int n = p.num_kv_heads * D;
    if (p.vec_v) {
      for (int i = threadIdx.x; i < n / 8; i += kRopeThreads)
        reinterpret_cast<uint4*>(vdst)[i] = reinterpret_cast<const uint4*>(vsrc)[i];
    } else {
      for (int i = threadIdx.x; i < n; i += kRopeThreads) vdst[i] = vsrc[i];
    }
  }
}

template <class Tag>
bool launch_rope(const RopeParams& p, int64_t num_tokens, int head_dim, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(num_tokens));
  if (head_dim == 128) {
    hipLaunchKernelGGL((qk_norm_rope_cache_kernel<Tag, 128>), grid, dim3(kRopeThreads), 0, s, p);
    return true;
  }
  if (head_dim == 64) {
    hipLaunchKernelGGL((qk_norm_rope_cache_kernel<Tag, 64>), grid, dim3(kRopeThreads), 0, s, p);
    return true;
  }
  return false;
}

}  // namespace

extern "C" void qk_norm_rope_and_cache(void* q_out, void* k_out, const void* qkv, int64_t qkv_row_stride,
                                       const void* q_norm_weight, const void* k_norm_weight, double eps,
                                       const float* cos_sin_cache, int64_t max_position,
                                       const int32_t* positions, void* key_cache, void* value_cache,
                                       const int64_t* slot_mapping, int64_t num_tokens, int64_t num_heads,
                                       int64_t num_kv_heads, int64_t head_dim, int dtype, void* stream) {
  if (dtype != OXIDE_DTYPE_BF16 && dtype != OXIDE_DTYPE_F16) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_DTYPE);
    return;
  }
  if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_tokens > INT32_MAX ||
      num_heads + num_kv_heads > 4096 || max_position <= 0 || max_position > INT32_MAX ||
      qkv_row_stride < (num_heads + 2 * num_kv_heads) * head_dim) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  if (head_dim != 64 && head_dim != 128) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_SHAPE);
    return;
  }
  if (num_tokens == 0) return;
  if (!q_out || !qkv || !cos_sin_cache || !positions ||
      (slot_mapping && (!key_cache || !value_cache))) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  RopeParams p{};
  p.q_out = static_cast<uint16_t*>(q_out);
  p.k_out = static_cast<uint16_t*>(k_out);
  p.qkv = static_cast<const uint16_t*>(qkv);
  p.q_weight = static_cast<const uint16_t*>(q_norm_weight);
  p.k_weight = static_cast<const uint16_t*>(k_norm_weight);
  p.cos_sin = cos_sin_cache;
  p.positions = positions;
  p.key_cache = static_cast<uint16_t*>(key_cache);
  p.value_cache = static_cast<uint16_t*>(value_cache);
  p.slot_mapping = slot_mapping;
  p.qkv_stride = qkv_row_stride;
  p.max_position = static_cast<int>(max_position);
  p.num_heads = static_cast<int>(num_heads);
  p.num_kv_heads = static_cast<int>(num_kv_heads);
  p.eps = static_cast<float>(eps);
  // The v part of every row starts at (Hq + Hkv) * D elements; 16-byte copies
  // need it, the row stride and the cache to be 16-byte aligned.
  p.vec_v = oxide::aligned16(qkv) && oxide::aligned16(value_cache) && (qkv_row_stride * 2) % 16 == 0 &&
            ((num_heads + num_kv_heads) * head_dim * 2) % 16 == 0 && (num_kv_heads * head_dim) % 8 == 0;
  hipStream_t s = oxide::as_stream(stream);
  const bool ok = dtype == OXIDE_DTYPE_BF16 ? launch_rope<Bf16Tag>(p, num_tokens, static_cast<int>(head_dim), s)
                                            : launch_rope<F16Tag>(p, num_tokens, static_cast<int>(head_dim), s);
  if (!ok) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_SHAPE);
    return;
  }
  oxide::check_launch();
}
