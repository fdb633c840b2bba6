/*
 * oxide_workload.h — host-side synthetic data for the benchmark workloads.
 *
 * No counterpart in the reference's paged-KV path (its own synthetic-input
 * tooling draws from a seeded generator as well).  One generator serves the
 * GPU run and the CPU baseline, so both see the same bytes: the caller fills a
 * host buffer once and uploads it.
 */
#ifndef OXIDE_WORKLOAD_H
#define OXIDE_WORKLOAD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Fills dst (host memory, n elements of dtype 0 = f16, 1 = bf16, 2 = f32) with
 * N(0, 1) samples.  Element pair (2i, 2i+1) comes from one 64-bit draw of a
 * counter-based generator, r = splitmix64(key + i * 0x9E3779B97F4A7C15) with
 * key = splitmix64(seed) ^ splitmix64(stream ^ 0xD1B54A32D192ED03), whose top 24
 * bits give u1 in (0, 1] and the next 24 bits u2 in [0, 1); Box-Muller in fp32
 * (sqrt(-2 ln u1) times cos / sin of 2 pi u2) gives the pair, rounded to the
 * dtype to nearest even.  The result depends on (seed, stream, n) only, not on
 * `threads` (<= 0: one per hardware thread).  Returns 0, or 1 for a bad argument.
 */
int oxide_fill_normal(void* dst, int64_t n, uint64_t seed, uint64_t stream, int dtype, int threads);

#ifdef __cplusplus
}
#endif

#endif /* OXIDE_WORKLOAD_H */
