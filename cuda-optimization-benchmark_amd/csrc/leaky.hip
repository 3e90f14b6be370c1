// leaky on gfx950: leaky integrate-and-fire layer (snnTorch Leaky, reset by subtraction).
//
// Drop-in signature tasks/leaky/tests/task.json:3, replacing
// reference/leaky/solution.cu:106-138.  The kernel is in leaky.hpp; the launch shape
// below is the measured best on MI355X.
#include "leaky.hpp"

namespace taskops {
namespace {
constexpr int kThreads = 256;
constexpr int kDepth = 16;
constexpr bool kNonTemporal = true;
}  // namespace
}  // namespace taskops

using namespace taskops;

extern "C" hipError_t taskops_leaky(const float* input_current, const float* mem0,
                                    const float* beta, const float* threshold, int32_t T,
                                    int32_t B, int32_t H, float* spikes, float* final_mem,
                                    hipStream_t stream) {
  if (T < 0 || B < 0 || H < 0) return hipErrorInvalidValue;
  const int64_t N = (int64_t)B * H;
  if (N == 0) return hipSuccess;
  const uintptr_t bits = reinterpret_cast<uintptr_t>(input_current) |
                         reinterpret_cast<uintptr_t>(spikes);
  int vec = 1;
  if (H % 2 == 0 && (bits & 7) == 0) vec = 2;
  const int64_t threads = N / vec;
  // One launch covers at most 2^32 - 1 work-items: B*H up to 2^32 - 256 neurons on either path.
  if (N > (int64_t(1) << 32) - kThreads) return hipErrorInvalidValue;
  const unsigned blocks = (unsigned)((threads + kThreads - 1) / kThreads);
  if (vec == 2)
    hipLaunchKernelGGL((leaky_kernel<kThreads, 2, kDepth, kNonTemporal>), dim3(blocks), dim3(kThreads), 0,
                       stream, input_current, mem0, beta, threshold, (int)T, N, (int)H, spikes, final_mem);
  else
    hipLaunchKernelGGL((leaky_kernel<kThreads, 1, kDepth, kNonTemporal>), dim3(blocks), dim3(kThreads), 0,
                       stream, input_current, mem0, beta, threshold, (int)T, N, (int)H, spikes, final_mem);
  return hipGetLastError();
}
