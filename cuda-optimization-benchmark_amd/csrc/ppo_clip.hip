// ppo_clip on gfx950: PPO clipped objective and its five diagnostics in one pass.
//
// Drop-in signature tasks/ppo_clip/tests/task.json:3, replacing
// reference/ppo_clip/solution.cu:165-182.  The entropy variant adds TorchRL
// ClipPPOLoss's entropy bonus (mean entropy and -coef * mean entropy).  The kernel is in
// ppo_clip.hpp; the launch shape below is the measured best on MI355X.
#include <mutex>

#include "ppo_clip.hpp"

// Scratch of taskops_ppo_clip_entropy_noalloc: the records and arrival counters of one
// reduction (PpoWorkspace's layout, 263,232 bytes per GPU, held until the process ends),
// in device memory that the code object brings with it, so that entry point allocates
// nothing.  In host code `scratch` names a host-side stand-in, not the device array:
// kernels and fills get the device address that hipGetSymbolAddress returns for it,
// looked up once per device with that device current (scratch_slots below).
static __device__ __align__(256) unsigned char scratch[sizeof(taskops::PpoWorkspace)];

namespace taskops {
namespace {

constexpr int kThreads = 512;
constexpr int kUnroll = 2;
constexpr int kBlocksPerCU = 1;
constexpr bool kNonTemporal = true;
// Samples per call at most: 2^40 (4 TiB per fp32 stream, far beyond one GPU's memory).
// Bounds B*T*H so the product cannot overflow int64.
constexpr int64_t kMaxSamples = int64_t(1) << 40;

// Where one launch publishes its per-workgroup records and counts its arrivals.
struct ReductionSlots {
  double (*records)[8];
  Arrivals* arrivals;
};

template <bool kEntropy>
hipError_t launch(int32_t B, int32_t T, int32_t H, const float* cur, const float* old,
                  const float* adv, const float* ent, float eps, float coef, float* out,
                  ReductionSlots slots, hipStream_t stream) {
  const int64_t n = (int64_t)B * T * H;
  PpoParams p;
  p.lo = log1p(-(double)eps);
  p.hi = log1p((double)eps);
  p.lo_ratio = (float)(1.0 - (double)eps);
  p.hi_ratio = (float)(1.0 + (double)eps);
  uintptr_t bits = reinterpret_cast<uintptr_t>(cur) | reinterpret_cast<uintptr_t>(old) |
                   reinterpret_cast<uintptr_t>(adv);
  if (kEntropy) bits |= reinterpret_cast<uintptr_t>(ent);
  const bool vec = (bits & 15) == 0;
  const int blocks = ppo_grid(n, kThreads, kUnroll, vec, device_cu_count(), kBlocksPerCU);
  if (vec)
    hipLaunchKernelGGL((ppo_clip_kernel<kThreads, kUnroll, true, kEntropy, kNonTemporal>), dim3(blocks),
                       dim3(kThreads), 0, stream, n, cur, old, adv, ent, p, coef, slots.records,
                       slots.arrivals, out);
  else
    hipLaunchKernelGGL((ppo_clip_kernel<kThreads, kUnroll, false, kEntropy, kNonTemporal>), dim3(blocks),
                       dim3(kThreads), 0, stream, n, cur, old, adv, ent, p, coef, slots.records,
                       slots.arrivals, out);
  return hipGetLastError();
}

hipError_t check_sizes(int32_t B, int32_t T, int32_t H) {
  if (B <= 0 || T <= 0 || H <= 0) return hipErrorInvalidValue;
  if ((int64_t)B * T > kMaxSamples / H) return hipErrorInvalidValue;
  return hipSuccess;
}

// The cached workspace of the allocating entry points.
hipError_t cached_slots(hipStream_t stream, ReductionSlots* slots) {
  void* wsp = nullptr;
  hipError_t e = workspace(kSlotPpo, sizeof(PpoWorkspace), stream, &wsp);
  if (e != hipSuccess) return e;
  auto* ws = static_cast<PpoWorkspace*>(wsp);
  *slots = {ws->partial, &ws->arrivals};
  return hipSuccess;
}

// The no-allocation entry point's scratch, per device.  One record per workgroup: the grid
// (ppo_grid) never exceeds PpoWorkspace::kMaxBlocks records, so any B*T*H up to
// kMaxSamples fits the fixed scratch.
constexpr size_t kScratchBytes = sizeof(PpoWorkspace);
static_assert(sizeof(::scratch) == kScratchBytes, "scratch holds one PpoWorkspace");
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

__global__ void clear_scratch(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    p[i] = uint4{0u, 0u, 0u, 0u};
}

// The current device's scratch address.  The first call on a device looks it up and
// clears the scratch with a kernel on `stream` (the arrival counters must start at zero;
// every launch leaves them zero again).  A stream of another device is refused.
hipError_t scratch_slots(hipStream_t stream, ReductionSlots* slots) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  if (stream != nullptr) {
    hipDevice_t sdev = 0;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return e;
    if (sdev != dev) return hipErrorInvalidValue;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(::scratch));
    if (e != hipSuccess) return e;
    if (ptr == nullptr) return hipErrorInvalidSymbol;
    static_assert(kScratchBytes % 16 == 0, "scratch is cleared in 16-byte words");
    hipLaunchKernelGGL(clear_scratch, dim3(64), dim3(256), 0, stream, static_cast<uint4*>(ptr),
                       kScratchBytes / 16);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    g_scratch[dev] = ptr;
  }
  auto* ws = static_cast<PpoWorkspace*>(g_scratch[dev]);
  *slots = {ws->partial, &ws->arrivals};
  return hipSuccess;
}

}  // namespace
}  // namespace taskops

extern "C" hipError_t taskops_ppo_clip(int32_t B, int32_t T, int32_t H,
                                       const float* current_log_prob, const float* old_log_prob,
                                       const float* advantage, float clip_epsilon, float* output,
                                       hipStream_t stream) {
  hipError_t e = taskops::check_sizes(B, T, H);
  if (e != hipSuccess) return e;
  taskops::ReductionSlots slots;
  e = taskops::cached_slots(stream, &slots);
  if (e != hipSuccess) return e;
  return taskops::launch<false>(B, T, H, current_log_prob, old_log_prob, advantage, nullptr,
                                clip_epsilon, 0.0f, output, slots, stream);
}

extern "C" hipError_t taskops_ppo_clip_entropy(int32_t B, int32_t T, int32_t H,
                                               const float* current_log_prob,
                                               const float* old_log_prob, const float* advantage,
                                               const float* entropy, float clip_epsilon,
                                               float entropy_coef, float* output,
                                               hipStream_t stream) {
  hipError_t e = taskops::check_sizes(B, T, H);
  if (e != hipSuccess) return e;
  taskops::ReductionSlots slots;
  e = taskops::cached_slots(stream, &slots);
  if (e != hipSuccess) return e;
  return taskops::launch<true>(B, T, H, current_log_prob, old_log_prob, advantage, entropy,
                               clip_epsilon, entropy_coef, output, slots, stream);
}

extern "C" hipError_t taskops_ppo_clip_entropy_noalloc(int32_t B, int32_t T, int32_t H,
                                                       const float* current_log_prob,
                                                       const float* old_log_prob,
                                                       const float* advantage,
                                                       const float* entropy, float clip_epsilon,
                                                       float entropy_coef, float* output,
                                                       hipStream_t stream) {
  hipError_t e = taskops::check_sizes(B, T, H);
  if (e != hipSuccess) return e;
  taskops::ReductionSlots slots;
  e = taskops::scratch_slots(stream, &slots);
  if (e != hipSuccess) return e;
  return taskops::launch<true>(B, T, H, current_log_prob, old_log_prob, advantage, entropy,
                               clip_epsilon, entropy_coef, output, slots, stream);
}
