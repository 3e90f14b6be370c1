// reward_to_go on gfx950: batched discounted reward-to-go with done flags.
//
// Drop-in signature tasks/reward_to_go/tests/task.json:3, replacing
// reference/reward_to_go/solution.cu:237-264.  The kernel is in reward_to_go.hpp.  Launch
// shape, measured on MI355X at B = T = 4096 (cold, µs per call): one workgroup per row;
// lanes own 4 steps, so every load and store instruction of a wave covers 1 KiB of
// contiguous memory; 4 waves of 4 chunks each cover 4096 steps, a BASELINE row in one
// segment; loads and stores are non-temporal.  That is 27.4 us against 30.5 us for 8 waves
// of one 8-step-per-lane chunk (whose 16-byte accesses cover every other 16 bytes per
// instruction, and which slows to 39 us with non-temporal stores).  Shorter rows use fewer
// waves and chunks per wave, so no wave idles.
#include "reward_to_go.hpp"

namespace taskops {
namespace {

constexpr int kPerLane = 4;
constexpr int kNonTemporal = 5;  // non-temporal loads (bit 0) and stores (policy 2 in bits 1-2)

// Rows of 4 waves x 4 chunks (T > 2048) run with at most this many workgroups per CU,
// held there by the LDS each one reserves (the kernel's own LDS is a few bytes).  At the
// kernel's 68 VGPRs the registers allow 7; 4 measured fastest at B = T = 4096 (25.53
// against 25.76 us per call, 5 and 6 slower, 3 slower still) and at B = 3000 (20.15 against
// 20.63 us), and the same at B = 8192 and 1024 (one MI355X, cold rotating inputs).
constexpr int kLongRowWorkgroupsPerCU = 4;

// Dynamic LDS that lets at most `per_cu` workgroups share a CU: more than 1/(per_cu+1) of it.
size_t occupancy_lds(int per_cu) { return (size_t)device_lds_per_cu() / (per_cu + 1) + 1; }

// One workgroup per row, and one launch covers at most 2^32 - 1 work-items in a dimension,
// so rows go out in launches of at most kRowsPerLaunch (one launch for every B up to it).
constexpr int kRowsPerLaunch = 1 << 23;

template <int kWaves, int kSeg>
void launch(const float* reward, const uint8_t* done, double g, int B, int T, float* out,
            bool vec, hipStream_t stream) {
  const size_t lds = (kWaves == 4 && kSeg == 4) ? occupancy_lds(kLongRowWorkgroupsPerCU) : 0;
  for (int b0 = 0; b0 < B; b0 += kRowsPerLaunch) {
    const int nb = B - b0 < kRowsPerLaunch ? B - b0 : kRowsPerLaunch;
    const size_t off = (size_t)b0 * (size_t)T;  // T % 4 == 0 on the vector path: alignment kept
    if (vec)
      hipLaunchKernelGGL((reward_to_go_kernel<kWaves, kPerLane, kSeg, true, kNonTemporal>), dim3(nb),
                         dim3(kWaves * kWave), lds, stream, reward + off, done + off, g, nb, T, out + off);
    else
      hipLaunchKernelGGL((reward_to_go_kernel<kWaves, kPerLane, kSeg, false, kNonTemporal>), dim3(nb),
                         dim3(kWaves * kWave), lds, stream, reward + off, done + off, g, nb, T, out + off);
  }
}

}  // namespace
}  // namespace taskops

using namespace taskops;

extern "C" hipError_t taskops_reward_to_go(const float* reward, const bool* done, float gamma,
                                           int32_t B, int32_t T, float* output,
                                           hipStream_t stream) {
  if (B <= 0 || T <= 0) return hipSuccess;  // nothing to write
  const uint8_t* d = reinterpret_cast<const uint8_t*>(done);
  // The vector path's buffer stores address a row in 32-bit bytes (store_row16).
  const bool vec = (T % 4) == 0 && T < (1 << 30) &&
                   ((reinterpret_cast<uintptr_t>(reward) | reinterpret_cast<uintptr_t>(output)) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(d) & 3) == 0;
  const int nchunks = (T + kWave * kPerLane - 1) / (kWave * kPerLane);  // chunks of 256 steps
  const double g = (double)gamma;
  if (nchunks <= 1)
    launch<1, 1>(reward, d, g, B, T, output, vec, stream);
  else if (nchunks <= 2)
    launch<2, 1>(reward, d, g, B, T, output, vec, stream);
  else if (nchunks <= 4)
    launch<4, 1>(reward, d, g, B, T, output, vec, stream);
  else if (nchunks <= 8)
    launch<4, 2>(reward, d, g, B, T, output, vec, stream);
  else
    launch<4, 4>(reward, d, g, B, T, output, vec, stream);
  return hipGetLastError();
}
