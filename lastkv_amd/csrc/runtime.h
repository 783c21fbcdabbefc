// Host-side status helpers shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>

#include "../../include/lastkv_amd.h"

namespace lkv {

// Records a thread-local message and returns `status`.
int32_t fail(int32_t status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks the launch that was just issued on this thread.
int32_t check_launch(const char* what);

inline hipStream_t as_stream(lkv_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

void clear_error();

// Compute units of the current device (cached per device); 0 when the query fails.
int device_cu_count();

}  // namespace lkv

#define LKV_REQUIRE(cond, ...)                                       \
  do {                                                               \
    if (!(cond)) return ::lkv::fail(LKV_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)
