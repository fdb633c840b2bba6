// Host-side N(0, 1) generator for the benchmark workloads (oxide_workload.h).
// Counter-based, so any split of the work over threads gives the same bytes.
#include "oxide_workload.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

inline uint16_t to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);  // round to nearest even (finite inputs)
  return static_cast<uint16_t>(u >> 16);
}

inline uint16_t to_f16(float f) {
  const _Float16 h = static_cast<_Float16>(f);
  uint16_t u;
  std::memcpy(&u, &h, 2);
  return u;
}

void fill_range(void* dst, int64_t n, uint64_t key, int dtype, int64_t p0, int64_t p1) {
  constexpr float kTwoPi = 6.2831853071795864769f;
  for (int64_t i = p0; i < p1; ++i) {
    const uint64_t r = splitmix64(key + static_cast<uint64_t>(i) * 0x9E3779B97F4A7C15ull);
    const float u1 = static_cast<float>((r >> 40) + 1) * 0x1p-24f;          // (0, 1]
    const float u2 = static_cast<float>((r >> 16) & 0xFFFFFFu) * 0x1p-24f;  // [0, 1)
    const float rad = std::sqrt(-2.0f * std::log(u1));
    const float z[2] = {rad * std::cos(kTwoPi * u2), rad * std::sin(kTwoPi * u2)};
    for (int k = 0; k < 2; ++k) {
      const int64_t e = 2 * i + k;
      if (e >= n) break;
      if (dtype == 1)
        static_cast<uint16_t*>(dst)[e] = to_bf16(z[k]);
      else if (dtype == 0)
        static_cast<uint16_t*>(dst)[e] = to_f16(z[k]);
      else
        static_cast<float*>(dst)[e] = z[k];
    }
  }
}

}  // namespace

extern "C" int oxide_fill_normal(void* dst, int64_t n, uint64_t seed, uint64_t stream, int dtype, int threads) {
  if (n < 0 || (n > 0 && dst == nullptr) || dtype < 0 || dtype > 2) return 1;
  const uint64_t key = splitmix64(seed) ^ splitmix64(stream ^ 0xD1B54A32D192ED03ull);
  const int64_t pairs = (n + 1) / 2;
  int t = threads > 0 ? threads : static_cast<int>(std::max(1u, std::thread::hardware_concurrency()));
  t = static_cast<int>(std::min<int64_t>(t, std::max<int64_t>(1, pairs / 65536)));
  if (t <= 1) {
    fill_range(dst, n, key, dtype, 0, pairs);
    return 0;
  }
  std::vector<std::thread> pool;
  for (int j = 0; j < t; ++j)
    pool.emplace_back(fill_range, dst, n, key, dtype, pairs * j / t, pairs * (j + 1) / t);
  for (auto& th : pool) th.join();
  return 0;
}
