// Host runtime of libtaskops: per-device cached workspaces and device facts.
#include <mutex>
#include <vector>

#include "common.hpp"

namespace taskops {
namespace {

constexpr int kMaxDevices = 64;

struct Region {
  void* ptr = nullptr;
  size_t bytes = 0;
};

std::mutex g_mu;
Region g_regions[kMaxDevices][kNumSlots];
// Buffers replaced by a larger one stay allocated until exit: a kernel enqueued before
// the replacement may still be using them, and freeing would need a host sync.
std::vector<void*> g_retired;
int g_cus[kMaxDevices] = {0};
int g_lds_per_cu[kMaxDevices] = {0};

// Zero fill as a kernel rather than hipMemsetAsync: no library call enqueues memset work,
// which keeps memset nodes out of any graph a caller captures.
__global__ void zero_fill(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    p[i] = uint4{0u, 0u, 0u, 0u};
}

}  // namespace

hipError_t workspace(WorkspaceSlot slot, size_t bytes, hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  // The workspace is the current device's; kernels run on the stream's device.  A stream of
  // another device is refused rather than handed memory it cannot use.
  if (stream != nullptr) {
    hipDevice_t sdev = 0;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return e;
    if (sdev != dev) return hipErrorInvalidValue;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  Region& r = g_regions[dev][slot];
  if (r.bytes < bytes) {
    const size_t want = ((bytes < 4096 ? 4096 : bytes) + 15) / 16 * 16;
    void* p = nullptr;
    e = hipMalloc(&p, want);
    if (e != hipSuccess) return e;
    const size_t n16 = want / 16;
    const unsigned blocks = (unsigned)(n16 / 256 < 4096 ? (n16 + 255) / 256 : 4096);
    hipLaunchKernelGGL(zero_fill, dim3(blocks), dim3(256), 0, stream, static_cast<uint4*>(p), n16);
    e = hipGetLastError();
    if (e != hipSuccess) {
      (void)hipFree(p);
      return e;
    }
    if (r.ptr) g_retired.push_back(r.ptr);
    r.ptr = p;
    r.bytes = want;
  }
  *out = r.ptr;
  return hipSuccess;
}

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = __atomic_load_n(&g_cus[dev], __ATOMIC_RELAXED);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  __atomic_store_n(&g_cus[dev], n, __ATOMIC_RELAXED);
  return n;
}

int device_lds_per_cu() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 160 * 1024;
  int n = __atomic_load_n(&g_lds_per_cu[dev], __ATOMIC_RELAXED);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess || n <= 0)
    n = 160 * 1024;
  __atomic_store_n(&g_lds_per_cu[dev], n, __ATOMIC_RELAXED);
  return n;
}

}  // namespace taskops

extern "C" int taskops_version(void) { return 1; }
