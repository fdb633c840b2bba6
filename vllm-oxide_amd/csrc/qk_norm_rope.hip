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
// Work split: a task is one head of one token -- a q head, a k head (norm +
// rotation) or a v head (copy) -- handled by D / 16 lanes (8 at D = 128);
// tasks are numbered token-major and walked by a resident grid (16 workgroups
// per CU) in a grid-stride loop that loads the next task's row slices before
// working on the current one.  Lane i of a q/k task holds elements
// [8 i, 8 i + 8) of each half, so the rotation partners x1[j] and x2[j] sit in
// the same lane and every access is 16 bytes (per element, in a second build
// of the kernel, when a row or weight is not 16-byte aligned).
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "cdna4_tile.hpp"
#include "exact_div.hpp"
#include "oxide_common.hpp"

namespace {

constexpr int kRopeThreads = 256;
template <int D>
constexpr int kLanesPerHead = D / 16;  // 8 elements of each half per lane

__device__ __forceinline__ float to_f32(Bf16Tag, uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }
__device__ __forceinline__ float to_f32(F16Tag, uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
// The low and high 16-bit values of a packed word, widened to fp32.
__device__ __forceinline__ float lo_f32(Bf16Tag, uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(Bf16Tag, uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float lo_f32(F16Tag, uint32_t w) { return to_f32(F16Tag{}, static_cast<uint16_t>(w)); }
__device__ __forceinline__ float hi_f32(F16Tag, uint32_t w) { return to_f32(F16Tag{}, static_cast<uint16_t>(w >> 16)); }

// x * w for two 16-bit values widened to fp32 (an exact product).  The empty asm
// keeps the compiler from fusing the multiply with the following round to f16
// into v_fma_mix with a +0 addend, which turns a -0 product into +0.
__device__ __forceinline__ float weigh(float x, float w) {
  float p = x * w;
  asm("" : "+v"(p));
  return p;
}

// Round a pair to the 16-bit type (nearest even, one packed convert for bf16)
// and widen it back: the reference's "to dtype" steps between fp32 operations.
template <class Tag>
__device__ __forceinline__ void round_pair(float& a, float& b) {
  const uint32_t u = pack2(Tag{}, a, b);
  a = to_f32(Tag{}, static_cast<uint16_t>(u));
  b = to_f32(Tag{}, static_cast<uint16_t>(u >> 16));
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
  int64_t num_tokens;
  float eps;
  bool vec;  // every row, head slice and weight 16-byte aligned: the vector-access kernel
};

typedef uint4 vec_t;  // 8 16-bit values
constexpr int E = 8;   // elements of each half per lane

// The qkv rows are read once: non-temporal loads keep them from displacing
// cached lines.  q, k and v are stored with the default policy (attention reads
// q next); non-temporal stores measured 3-4 us slower at 16k tokens.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ vec_t load_row16(const uint16_t* p) {
  return __builtin_bit_cast(vec_t, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
}
__device__ __forceinline__ void store_row16(uint16_t* p, vec_t v) {
  *reinterpret_cast<vec_t*>(p) = v;
}

// One task's inputs: its token and head, the two 16-byte slices of its qkv
// head row this lane holds (elements [8 sub, 8 sub + 8) of each half), the
// token's position and cache slot.
struct TaskIn {
  int64_t t;
  int h;
  vec_t a, b;
  int pos;
  int64_t slot;
};

// Position-dependent and per-head-kind operands of a q / k task: the norm
// weight slices and the cos / sin values this lane multiplies by.
struct TaskSide {
  vec_t w1, w2;
  float c[E], s[E];
};

__device__ __forceinline__ void split_task(int64_t task, int heads, bool narrow, int64_t& t, int& h) {
  if (narrow) {  // a 64-bit divide is ~10x the cost of the 32-bit one
    t = static_cast<uint32_t>(task) / static_cast<uint32_t>(heads);
    h = static_cast<int>(static_cast<uint32_t>(task) - static_cast<uint32_t>(t) * heads);
  } else {
    t = task / heads;
    h = static_cast<int>(task - t * heads);
  }
}

// `real` false: a lane with no further task -- the row loads still issue (the
// waits stay exact) but read the norm weight row (or the cos / sin table),
// which every task reads with ordinary loads and so sits in L2: re-reading the
// current task's row would fetch it from HBM again, since the row loads are
// non-temporal and do not keep their lines.
template <int D, bool V>
__device__ __forceinline__ void load_task(const RopeParams& p, int64_t task, int heads, bool narrow, TaskIn& in,
                                          bool real = true) {
  constexpr int LPH = kLanesPerHead<D>;
  const int sub = threadIdx.x % LPH;
  split_task(task, heads, narrow, in.t, in.h);
  // Position and slot first: the side loads wait on the position, not on the rows.
  in.pos = p.positions[in.t];
  // Unconditional (without a slot mapping it reads the cos / sin table and
  // discards the value): every path through the task loop then issues the same
  // loads, and the waits stay exact.
  const int64_t sv = *(p.slot_mapping ? p.slot_mapping + in.t : reinterpret_cast<const int64_t*>(p.cos_sin));
  in.slot = p.slot_mapping ? sv : -1;
  const uint16_t* stand_in = p.q_weight ? p.q_weight : reinterpret_cast<const uint16_t*>(p.cos_sin);
  const uint16_t* src = real ? p.qkv + in.t * p.qkv_stride + static_cast<int64_t>(in.h) * D : stand_in;
  if constexpr (V) {
    in.a = load_row16(src + sub * E);
    in.b = load_row16(src + D / 2 + sub * E);
  } else {
    uint16_t r1[E], r2[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      r1[e] = src[sub * E + e];
      r2[e] = src[D / 2 + sub * E + e];
    }
    __builtin_memcpy(&in.a, r1, sizeof(in.a));
    __builtin_memcpy(&in.b, r2, sizeof(in.b));
  }
}

template <int D, bool V>
__device__ __forceinline__ void load_side(const RopeParams& p, const TaskIn& in, TaskSide& sd) {
  constexpr int LPH = kLanesPerHead<D>;
  const int sub = threadIdx.x % LPH;
  const int pos = min(max(in.pos, 0), p.max_position - 1);
  const float* cs = p.cos_sin + static_cast<int64_t>(pos) * D;
  // Issued for every task (v heads and weightless norms read a stand-in row and
  // ignore it), so the loads counted in flight do not depend on the head kind.
  const uint16_t* w = in.h < p.num_heads ? p.q_weight : p.k_weight;
  if (w == nullptr) w = reinterpret_cast<const uint16_t*>(cs);
  {
    if constexpr (V) {
      sd.w1 = *reinterpret_cast<const vec_t*>(w + sub * E);
      sd.w2 = *reinterpret_cast<const vec_t*>(w + D / 2 + sub * E);
    } else {
      uint16_t w1[E], w2[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        w1[e] = w[sub * E + e];
        w2[e] = w[D / 2 + sub * E + e];
      }
      __builtin_memcpy(&sd.w1, w1, sizeof(sd.w1));
      __builtin_memcpy(&sd.w2, w2, sizeof(sd.w2));
    }
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    sd.c[e] = cs[sub * E + e];
    sd.s[e] = cs[D / 2 + sub * E + e];
  }
}

template <class Tag, int D, bool V>
__device__ __forceinline__ void rope_task(const RopeParams& p, const TaskIn& in, const TaskSide& sd) {
  // Every product and sum is rounded on its own, as in the reference.
#pragma clang fp contract(off)
  constexpr int LPH = kLanesPerHead<D>;
  const int sub = threadIdx.x % LPH;
  const int h = in.h;
  const int64_t t = in.t;
  const int64_t slot = in.slot;

  if (h >= p.num_heads + p.num_kv_heads) {
    // v head: bitwise copy into the slot (2 x 16 bytes per lane).
    if (slot < 0) return;
    uint16_t* dst = p.value_cache + (slot * p.num_kv_heads + (h - p.num_heads - p.num_kv_heads)) * D;
    if constexpr (V) {
      store_row16(dst + sub * E, in.a);
      store_row16(dst + D / 2 + sub * E, in.b);
    } else {
      uint16_t r1[E], r2[E];
      __builtin_memcpy(r1, &in.a, sizeof(in.a));
      __builtin_memcpy(r2, &in.b, sizeof(in.b));
#pragma unroll
      for (int e = 0; e < E; ++e) {
        dst[sub * E + e] = r1[e];
        dst[D / 2 + sub * E + e] = r2[e];
      }
    }
    return;
  }

  const bool is_q = h < p.num_heads;
  const bool has_w = (is_q ? p.q_weight : p.k_weight) != nullptr;
  const uint32_t ra[4] = {in.a.x, in.a.y, in.a.z, in.a.w}, rb[4] = {in.b.x, in.b.y, in.b.z, in.b.w};
  const uint32_t wa[4] = {sd.w1.x, sd.w1.y, sd.w1.z, sd.w1.w}, wb[4] = {sd.w2.x, sd.w2.y, sd.w2.z, sd.w2.w};

  float x1[E], x2[E];
#pragma unroll
  for (int e = 0; e < E; e += 2) {
    x1[e] = lo_f32(Tag{}, ra[e / 2]);
    x1[e + 1] = hi_f32(Tag{}, ra[e / 2]);
    x2[e] = lo_f32(Tag{}, rb[e / 2]);
    x2[e + 1] = hi_f32(Tag{}, rb[e / 2]);
  }
  if (has_w) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) ss = ss + (x1[e] * x1[e] + x2[e] * x2[e]);
#pragma unroll
    for (int m = 1; m < LPH; m <<= 1) ss = ss + __shfl_xor(ss, m);
    const float sd_ = sqrtf(ss / static_cast<float>(D) + p.eps);  // correctly rounded / and sqrt
    // x / sd correctly rounded: three operations per element against the
    // shared reciprocal where exact_div's domain holds (always, short of
    // extreme inputs), the general divide otherwise.
    bool fast = oxide::exact_div_divisor_ok(sd_);
#pragma unroll
    for (int e = 0; e < E; ++e)
      fast = fast & oxide::exact_div_dividend_ok(x1[e]) & oxide::exact_div_dividend_ok(x2[e]);
    if (fast) {
      const float y = 1.0f / sd_;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        x1[e] = oxide::exact_div(x1[e], sd_, y);
        x2[e] = oxide::exact_div(x2[e], sd_, y);
      }
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        x1[e] = x1[e] / sd_;
        x2[e] = x2[e] / sd_;
      }
    }
#pragma unroll
    for (int e = 0; e < E; e += 2) {
      round_pair<Tag>(x1[e], x1[e + 1]);
      round_pair<Tag>(x2[e], x2[e + 1]);
      x1[e] = weigh(x1[e], lo_f32(Tag{}, wa[e / 2]));
      x1[e + 1] = weigh(x1[e + 1], hi_f32(Tag{}, wa[e / 2]));
      x2[e] = weigh(x2[e], lo_f32(Tag{}, wb[e / 2]));
      x2[e + 1] = weigh(x2[e + 1], hi_f32(Tag{}, wb[e / 2]));
      round_pair<Tag>(x1[e], x1[e + 1]);
      round_pair<Tag>(x2[e], x2[e + 1]);
    }
  }
  uint32_t y1[E / 2], y2[E / 2];  // packed pairs
#pragma unroll
  for (int e = 0; e < E; e += 2) {
    y1[e / 2] = pack2(Tag{}, x1[e] * sd.c[e] - x2[e] * sd.s[e], x1[e + 1] * sd.c[e + 1] - x2[e + 1] * sd.s[e + 1]);
    y2[e / 2] = pack2(Tag{}, x2[e] * sd.c[e] + x1[e] * sd.s[e], x2[e + 1] * sd.c[e + 1] + x1[e + 1] * sd.s[e + 1]);
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
  for (uint16_t* dst : {dst0, dst1}) {
    if (dst == nullptr) continue;
    if constexpr (V) {
      vec_t a, b;
      __builtin_memcpy(&a, y1, sizeof(a));
      __builtin_memcpy(&b, y2, sizeof(b));
      store_row16(dst + sub * E, a);
      store_row16(dst + D / 2 + sub * E, b);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        dst[sub * E + e] = static_cast<uint16_t>(y1[e / 2] >> (16 * (e & 1)));
        dst[D / 2 + sub * E + e] = static_cast<uint16_t>(y2[e / 2] >> (16 * (e & 1)));
      }
    }
  }
}

// Grid-stride over tasks with the next task's row loads issued before this
// task's arithmetic: each lane keeps two tasks' 32 bytes in flight.  The
// weights and cos / sin of the current task are issued before the prefetch,
// since loads complete in issue order and waiting on them must not wait on it.
// Five waves per SIMD (96 VGPRs, no spills; the unconstrained build took 97 and so four
// waves): 73.5 -> 72.6 us at 16k tokens, bit-identical; six or eight spill.
template <class Tag, int D, bool V>
__global__ __launch_bounds__(kRopeThreads) __attribute__((amdgpu_waves_per_eu(5, 5)))
void qk_norm_rope_cache_kernel(RopeParams p) {
  const int heads = p.num_heads + 2 * p.num_kv_heads;  // q, k, v heads per token
  constexpr int kTasksPerWg = kRopeThreads / kLanesPerHead<D>;
  const int64_t tasks = p.num_tokens * heads;
  int64_t task = static_cast<int64_t>(blockIdx.x) * kTasksPerWg + threadIdx.x / kLanesPerHead<D>;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kTasksPerWg;
  const bool narrow = tasks <= INT32_MAX;
  if (task >= tasks) return;
  // Two task slots used in turn, so no register copy of a pending load is needed.
  TaskIn ta, tb;
  load_task<D, V>(p, task, heads, narrow, ta);
  while (true) {
    TaskSide sd;
    load_side<D, V>(p, ta, sd);
    const int64_t nb = task + stride;
    const bool more_b = nb < tasks;
    load_task<D, V>(p, more_b ? nb : task, heads, narrow, tb, more_b);  // unconditional, as above
    rope_task<Tag, D, V>(p, ta, sd);
    if (!more_b) break;
    load_side<D, V>(p, tb, sd);
    const int64_t na = nb + stride;
    const bool more_a = na < tasks;
    load_task<D, V>(p, more_a ? na : nb, heads, narrow, ta, more_a);
    rope_task<Tag, D, V>(p, tb, sd);
    if (!more_a) break;
    task = na;
  }
}

// Resident workgroups per CU of the prologue grid.
constexpr int kRopeWgsPerCu = 16;
template <class Tag>
bool launch_rope(const RopeParams& p, int64_t num_tokens, int head_dim, hipStream_t s) {
  const int64_t tasks = num_tokens * (p.num_heads + 2 * p.num_kv_heads);
  const int tpw = kRopeThreads / (static_cast<int>(head_dim) / 16);  // tasks per workgroup
  const int64_t wgs = (tasks + tpw - 1) / tpw;
  // A resident grid: each lane walks several tasks, prefetching the next.
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(wgs, int64_t{kRopeWgsPerCu} * oxide::device_cu_count())));
  auto kernel = [&](auto d) {
    constexpr int D = decltype(d)::value;
    return p.vec ? qk_norm_rope_cache_kernel<Tag, D, true> : qk_norm_rope_cache_kernel<Tag, D, false>;
  };
  if (head_dim == 128) {
    hipLaunchKernelGGL(kernel(std::integral_constant<int, 128>{}), grid, dim3(kRopeThreads), 0, s, p);
    return true;
  }
  if (head_dim == 64) {
    hipLaunchKernelGGL(kernel(std::integral_constant<int, 64>{}), grid, dim3(kRopeThreads), 0, s, p);
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
  p.num_tokens = num_tokens;
  // Head slices are D * 2 bytes apart (a multiple of 16); vector accesses need
  // every base pointer (weights included) and the qkv row stride 16-byte aligned as well.
  auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; };
  p.vec = al16(qkv) && al16(q_out) && al16(k_out) && al16(key_cache) && al16(value_cache) &&
          al16(q_norm_weight) && al16(k_norm_weight) && al16(cos_sin_cache) && (qkv_row_stride * 2) % 16 == 0;
  hipStream_t s = oxide::as_stream(stream);
  const bool ok = dtype == OXIDE_DTYPE_BF16 ? launch_rope<Bf16Tag>(p, num_tokens, static_cast<int>(head_dim), s)
                                            : launch_rope<F16Tag>(p, num_tokens, static_cast<int>(head_dim), s);
  if (!ok) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_SHAPE);
    return;
  }
  oxide::check_launch();
}
