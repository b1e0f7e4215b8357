// Host-side helpers shared by the C-ABI entry points: argument checks, the
// per-thread error text, the gfx950 device check and launch-status collection.
#pragma once

#include <errno.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "omnia_hip.h"

namespace omnia {

// Records `message` as the calling thread's last error and returns `code`.
int32_t fail(int32_t code, const std::string& message);

// 0 when `stream` belongs to the current device and that device is a gfx950.
// A stream of another device gives -EINVAL, a device of another architecture
// -ENODEV (with the error text set). The null stream stands for the current
// device. The architecture is cached per device ordinal after the first query.
int32_t check_device(hipStream_t stream);

// Converts the status of the launch just made into the ABI's return code.
int32_t launched(const char* kernel);

inline bool aligned16(const void* ptr) {
  return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0;
}

}  // namespace omnia

#define OMNIA_REQUIRE(cond, message)                         \
  do {                                                       \
    if (!(cond)) return ::omnia::fail(-EINVAL, (message));   \
  } while (0)
