// Shared internals of the gfx950 paged-KV library: per-thread error state,
// dtype sizes and launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oxide_paged_kv.h"

namespace oxide {

// 128-bit vector of the native clang kind (usable with the nontemporal builtins).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Records `code` as the calling thread's error unless one is already pending.
void set_error(int code);

// Checks the launch just issued; records OXIDE_ERR_HIP + code on failure.
void check_launch();

// Compute units of the current device (cached per device; 256 when the query fails).
int device_cu_count();

// First-use device queries (CU counts, occupancies, the static scratch's address)
// run inside this scope: the calling thread's stream-capture mode is relaxed for its
// lifetime, so a first call made under HIP graph capture (global mode) may query the
// device -- the queries enqueue nothing on any stream.
struct RelaxedCaptureScope {
  hipStreamCaptureMode saved = hipStreamCaptureModeRelaxed;
  bool ok;
  RelaxedCaptureScope() : ok(hipThreadExchangeStreamCaptureMode(&saved) == hipSuccess) {}
  ~RelaxedCaptureScope() {
    if (ok) (void)hipThreadExchangeStreamCaptureMode(&saved);
  }
  RelaxedCaptureScope(const RelaxedCaptureScope&) = delete;
  RelaxedCaptureScope& operator=(const RelaxedCaptureScope&) = delete;
};

inline int dtype_size(int dtype) {
  switch (dtype) {
    case OXIDE_DTYPE_F16:
    case OXIDE_DTYPE_BF16:
      return 2;
    case OXIDE_DTYPE_F32:
      return 4;
    default:
      return 0;
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace oxide
