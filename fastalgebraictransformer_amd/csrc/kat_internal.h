// Host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kat.h"

namespace kat {

// Record a failure message for kat_last_error() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Turn the launch status of the kernel just enqueued into a kat_status.
int check_launch(const char* what);

// Compute units of the current device (cached per device).
int num_cus();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int dtype_size(int dtype) {
  switch (dtype) {
    case KAT_F32: return 4;
    case KAT_BF16: return 2;
    case KAT_F16: return 2;
    case KAT_F64: return 8;
    default: return 0;
  }
}

}  // namespace kat
