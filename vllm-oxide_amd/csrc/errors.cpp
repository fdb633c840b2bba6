// Per-host-thread error state behind oxide_last_error(), and the cached
// compute-unit count the launch policies size their grids by.  The reference's entry
// points return void and drop launch errors (reshape_and_cache.cu:30,
// copy_blocks.cu:30); this library keeps the void ABI and makes the failure
// queryable instead.
#include <atomic>

#include "oxide_common.hpp"

namespace oxide {

static thread_local int g_last_error = OXIDE_OK;

void set_error(int code) {
  if (g_last_error == OXIDE_OK) g_last_error = code;
}

void check_launch() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) set_error(OXIDE_ERR_HIP + static_cast<int>(e));
}

int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  std::atomic<int>& n = cache[dev % kMaxDevices];
  int v = n.load(std::memory_order_relaxed);
  if (v == 0) {
    RelaxedCaptureScope relaxed;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    n.store(v, std::memory_order_relaxed);
  }
  return v;
}

}  // namespace oxide

extern "C" int oxide_last_error(void) { return oxide::g_last_error; }

extern "C" void oxide_clear_error(void) { oxide::g_last_error = OXIDE_OK; }

extern "C" const char* oxide_error_string(int code) {
  switch (code) {
    case OXIDE_OK:
      return "ok";
    case OXIDE_ERR_INVALID_ARGUMENT:
      return "invalid argument";
    case OXIDE_ERR_UNSUPPORTED_DTYPE:
      return "unsupported dtype code";
    case OXIDE_ERR_UNSUPPORTED_SHAPE:
      return "unsupported shape (head_dim, group size or block size)";
    case OXIDE_ERR_WORKSPACE_TOO_SMALL:
      return "workspace too small";
    case OXIDE_ERR_SCRATCH_TOO_SMALL:
      return "shape needs more partial-result memory than the static scratch of "
             "paged_decode_attention_noalloc (48 MiB per device)";
    default:
      if (code > OXIDE_ERR_HIP) return hipGetErrorString(static_cast<hipError_t>(code - OXIDE_ERR_HIP));
      return "unknown error";
  }
}
