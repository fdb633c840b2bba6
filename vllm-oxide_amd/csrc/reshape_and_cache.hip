// KV append: scatter the step's new K/V rows into their paged-cache slots.
//
// Semantics follow crates/vllm-oxide/kernels/reshape_and_cache.cu:6-28 (row t
// of key/value lands at row slot_mapping[t] of the per-layer cache view; -1 is
// skipped) and the C entry at :30-71 (same symbol and parameters).  The copy
// is bitwise, so one kernel serves every dtype: only the row byte count
// matters.
//
// gfx950 design: one workgroup per token moves the token's K row and V row
// together (2 * H*D*esize bytes).  Rows whose byte count is a multiple of 16
// with 16-byte aligned tensors use 128-bit loads/stores (global_load_dwordx4),
// one vector per lane: at Qwen3 shapes (H*D = 1024 bf16 = 2 KiB per row) a
// 256-lane workgroup moves K and V in a single coalesced pass.  Anything else
// falls back to a per-element copy of the element's bit pattern.  At decode
// sizes (a few dozen tokens) the launch itself dominates; the kernel does one
// round trip of memory latency.
#include "oxide_common.hpp"

namespace {

__global__ __launch_bounds__(256) void append_rows_vec16(const uint4* __restrict__ key,
                                                         const uint4* __restrict__ value,
                                                         uint4* __restrict__ key_cache,
                                                         uint4* __restrict__ value_cache,
                                                         const int64_t* __restrict__ slot_mapping,
                                                         int64_t row_vecs) {
  const int64_t t = blockIdx.x;
  const int64_t slot = slot_mapping[t];
  if (slot < 0) return;
  const int64_t src_base = t * row_vecs;
  const int64_t dst_base = slot * row_vecs;
  // Lanes [0, row_vecs) copy K, lanes [row_vecs, 2*row_vecs) copy V.
  for (int64_t i = threadIdx.x; i < 2 * row_vecs; i += blockDim.x) {
    if (i < row_vecs) {
      key_cache[dst_base + i] = key[src_base + i];
    } else {
      const int64_t j = i - row_vecs;
      value_cache[dst_base + j] = value[src_base + j];
    }
  }
}

template <typename E>
__global__ __launch_bounds__(256) void append_rows_elem(const E* __restrict__ key,
                                                        const E* __restrict__ value,
                                                        E* __restrict__ key_cache,
                                                        E* __restrict__ value_cache,
                                                        const int64_t* __restrict__ slot_mapping,
                                                        int64_t row_elems) {
  const int64_t t = blockIdx.x;
  const int64_t slot = slot_mapping[t];
  if (slot < 0) return;
  for (int64_t e = threadIdx.x; e < row_elems; e += blockDim.x) {
    key_cache[slot * row_elems + e] = key[t * row_elems + e];
    value_cache[slot * row_elems + e] = value[t * row_elems + e];
  }
}

}  // namespace

extern "C" void reshape_and_cache(const void* key, const void* value, void* key_cache,
                                  void* value_cache, const int64_t* slot_mapping,
                                  int64_t num_tokens, int64_t num_kv_heads, int64_t head_dim,
                                  int dtype, void* stream) {
  const int esize = oxide::dtype_size(dtype);
  if (esize == 0) {
    oxide::set_error(OXIDE_ERR_UNSUPPORTED_DTYPE);
    return;
  }
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  if (num_tokens == 0) return;
  if (!key || !value || !key_cache || !value_cache || !slot_mapping || num_tokens > INT32_MAX) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  hipStream_t s = oxide::as_stream(stream);
  const int64_t row_elems = num_kv_heads * head_dim;
  const int64_t row_bytes = row_elems * esize;
  const dim3 grid(static_cast<unsigned>(num_tokens));
  if (row_bytes % 16 == 0 && oxide::aligned16(key) && oxide::aligned16(value) &&
      oxide::aligned16(key_cache) && oxide::aligned16(value_cache)) {
    const int64_t row_vecs = row_bytes / 16;
    int64_t threads = ((2 * row_vecs + 63) / 64) * 64;
    if (threads > 256) threads = 256;
    hipLaunchKernelGGL(append_rows_vec16, grid, dim3(static_cast<unsigned>(threads)), 0, s,
                       static_cast<const uint4*>(key), static_cast<const uint4*>(value),
                       static_cast<uint4*>(key_cache), static_cast<uint4*>(value_cache),
                       slot_mapping, row_vecs);
  } else {
    int64_t threads = ((row_elems + 63) / 64) * 64;
    if (threads > 256) threads = 256;
    const dim3 block(static_cast<unsigned>(threads));
    if (esize == 2) {
      hipLaunchKernelGGL(append_rows_elem<uint16_t>, grid, block, 0, s,
                         static_cast<const uint16_t*>(key), static_cast<const uint16_t*>(value),
                         static_cast<uint16_t*>(key_cache), static_cast<uint16_t*>(value_cache),
                         slot_mapping, row_elems);
    } else {
      hipLaunchKernelGGL(append_rows_elem<uint32_t>, grid, block, 0, s,
                         static_cast<const uint32_t*>(key), static_cast<const uint32_t*>(value),
                         static_cast<uint32_t*>(key_cache), static_cast<uint32_t*>(value_cache),
                         slot_mapping, row_elems);
    }
  }
  oxide::check_launch();
}
