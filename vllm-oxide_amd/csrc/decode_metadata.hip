// Device-side decode metadata: cu_seqlens_k and the slot of each sequence's
// new token, built on the GPU from context lengths and the padded block table.
//
// Semantics are the reference's decode-step preparation
// (crates/vllm-oxide/src/engine/mod.rs:247-267): for sequence b with
// L = context_lens[b] (the new token included),
//   cu_seqlens_k[b+1] = cu_seqlens_k[b] + L                   (metadata.rs:30-37)
//   slot_mapping[b]   = compute_slot_mapping(seq, L - 1, 1)   (kv_cache_manager.rs:115-135)
//                     = table[b][(L-1)/BS] * BS + (L-1) % BS, or -1 when that
//                       block index is past the row (>= max_blocks) or L == 0.
// The reference builds these on the host and uploads them in every layer; an
// engine that keeps context lengths and block tables on the device can run
// this once per step and feed every layer's append and attention from it.
//
// One workgroup of 1024 lanes: each lane sums a contiguous run of sequences,
// the run totals are scanned in LDS, and each lane writes its run's prefix
// sums and slots.  Batches of up to 65535 sequences.
#include "oxide_common.hpp"

namespace {

constexpr int kLanes = 1024;

__global__ __launch_bounds__(kLanes) void decode_metadata_kernel(const uint32_t* __restrict__ context_lens,
                                                                 const int32_t* __restrict__ block_table,
                                                                 int64_t max_blocks, int batch,
                                                                 int block_size,
                                                                 uint32_t* __restrict__ cu_seqlens_k,
                                                                 int64_t* __restrict__ slot_mapping) {
  __shared__ uint32_t s_sum[kLanes];
  const int t = threadIdx.x;
  const int per = (batch + kLanes - 1) / kLanes;
  const int b0 = t * per;
  const int b1 = min(batch, b0 + per);
  uint32_t run = 0;
  for (int b = b0; b < b1; ++b) run += context_lens[b];
  s_sum[t] = run;
  __syncthreads();
  // Inclusive Hillis-Steele scan of the run totals.
  for (int off = 1; off < kLanes; off <<= 1) {
    const uint32_t add = t >= off ? s_sum[t - off] : 0u;
    __syncthreads();
    s_sum[t] += add;
    __syncthreads();
  }
  uint32_t acc = s_sum[t] - run;  // exclusive prefix of this run
  if (t == 0) cu_seqlens_k[0] = 0;
  for (int b = b0; b < b1; ++b) {
    const uint32_t L = context_lens[b];
    acc += L;
    cu_seqlens_k[b + 1] = acc;
    int64_t slot = -1;
    if (L > 0) {
      const int64_t pos = static_cast<int64_t>(L) - 1;
      const int64_t blk = pos / block_size;
      if (blk < max_blocks)
        slot = static_cast<int64_t>(block_table[static_cast<int64_t>(b) * max_blocks + blk]) * block_size +
               pos % block_size;
    }
    slot_mapping[b] = slot;
  }
}

}  // namespace

extern "C" void build_decode_metadata_device(const uint32_t* context_lens, const int32_t* block_table,
                                             int64_t max_blocks_per_seq, int64_t batch,
                                             int64_t block_size, uint32_t* cu_seqlens_k,
                                             int64_t* slot_mapping, void* stream) {
  if (batch < 0 || max_blocks_per_seq < 0 || block_size <= 0 || batch > 65535 ||
      block_size > INT32_MAX) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  if (!cu_seqlens_k || (batch > 0 && (!context_lens || !slot_mapping ||
                                      (max_blocks_per_seq > 0 && !block_table)))) {
    oxide::set_error(OXIDE_ERR_INVALID_ARGUMENT);
    return;
  }
  hipLaunchKernelGGL(decode_metadata_kernel, dim3(1), dim3(kLanes), 0, oxide::as_stream(stream),
                     context_lens, block_table, max_blocks_per_seq, static_cast<int>(batch),
                     static_cast<int>(block_size), cu_seqlens_k, slot_mapping);
  oxide::check_launch();
}
