// reward_to_go on gfx950: batched discounted reward-to-go with done flags.
//
// Drop-in signature tasks/reward_to_go/tests/task.json:3, replacing
// reference/reward_to_go/solution.cu:237-264.  The kernel is in reward_to_go.hpp; the
// launch shape below is the measured best on MI355X: one workgroup per row, with as
// many waves (up to 8) as the row has chunks of 64*kPerLane steps.
#include "reward_to_go.hpp"

namespace taskops {
namespace {

constexpr int kPerLane = 8;
constexpr int kSeg = 1;
constexpr int kNonTemporal = 0;

template <int kWaves>
void launch(const float* reward, const uint8_t* done, double g, int B, int T, float* out,
            bool vec, hipStream_t stream) {
  if (vec)
    hipLaunchKernelGGL((reward_to_go_kernel<kWaves, kPerLane, kSeg, true, kNonTemporal>), dim3(B),
                       dim3(kWaves * kWave), 0, stream, reward, done, g, B, T, out);
  else
    hipLaunchKernelGGL((reward_to_go_kernel<kWaves, kPerLane, kSeg, false, kNonTemporal>), dim3(B),
                       dim3(kWaves * kWave), 0, stream, reward, done, g, B, T, out);
}

}  // namespace
}  // namespace taskops

using namespace taskops;

extern "C" hipError_t taskops_reward_to_go(const float* reward, const bool* done, float gamma,
                                           int32_t B, int32_t T, float* output,
                                           hipStream_t stream) {
  if (B <= 0 || T <= 0) return hipSuccess;  // nothing to write
  const uint8_t* d = reinterpret_cast<const uint8_t*>(done);
  const bool vec = (T % 4) == 0 &&
                   ((reinterpret_cast<uintptr_t>(reward) | reinterpret_cast<uintptr_t>(output)) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(d) & 3) == 0;
  const int nchunks = (T + kWave * kPerLane - 1) / (kWave * kPerLane);
  int waves = 1;
  while (waves < 8 && waves * kSeg < nchunks) waves *= 2;
  const double g = (double)gamma;
  switch (waves) {
    case 1: launch<1>(reward, d, g, B, T, output, vec, stream); break;
    case 2: launch<2>(reward, d, g, B, T, output, vec, stream); break;
    case 4: launch<4>(reward, d, g, B, T, output, vec, stream); break;
    default: launch<8>(reward, d, g, B, T, output, vec, stream); break;
  }
  return hipGetLastError();
}
