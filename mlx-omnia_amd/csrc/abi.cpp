// ABI bookkeeping: version, per-thread error text, device check.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <string>

#include "host.hpp"

namespace omnia {

namespace {

thread_local std::string last_error;

constexpr int kMaxDevices = 64;
// 0 = not yet queried, 1 = gfx950, 2 = some other architecture.
std::atomic<int> device_kind[kMaxDevices];

}  // namespace

int32_t fail(int32_t code, const std::string& message) {
  last_error = message;
  return code;
}

int32_t check_device(hipStream_t stream) {
  int device = 0;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) {
    return fail(-ENODEV, std::string("hipGetDevice: ") + hipGetErrorString(status));
  }
  if (stream != nullptr) {
    // The kernels run on the stream's device and dereference the caller's pointers
    // there; a stream of another device than the current one is a caller mistake.
    hipDevice_t owner = 0;
    status = hipStreamGetDevice(stream, &owner);
    if (status != hipSuccess) {
      return fail(-EINVAL, std::string("hipStreamGetDevice: ") + hipGetErrorString(status));
    }
    if (owner != device) {
      return fail(-EINVAL, "the stream belongs to device " + std::to_string(owner) +
                               " but device " + std::to_string(device) +
                               " is current; make the stream's device current first");
    }
  }
  if (device < 0 || device >= kMaxDevices) {
    return fail(-ENODEV, "device ordinal out of range");
  }
  int kind = device_kind[device].load(std::memory_order_acquire);
  if (kind == 0) {
    hipDeviceProp_t props;
    status = hipGetDeviceProperties(&props, device);
    if (status != hipSuccess) {
      return fail(-ENODEV, std::string("hipGetDeviceProperties: ") +
                               hipGetErrorString(status));
    }
    kind = std::strncmp(props.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
    device_kind[device].store(kind, std::memory_order_release);
  }
  if (kind != 1) {
    return fail(-ENODEV, "current device is not gfx950 (MI355X)");
  }
  return 0;
}

int32_t launched(const char* kernel) {
  hipError_t status = hipGetLastError();
  if (status != hipSuccess) {
    return fail(-1, std::string(kernel) + " launch failed: " + hipGetErrorString(status));
  }
  return 0;
}

}  // namespace omnia

extern "C" int32_t omnia_abi_version(void) { return OMNIA_ABI_VERSION; }

extern "C" const char* omnia_last_error(void) { return omnia::last_error.c_str(); }
