// ppo_clip on gfx950: PPO clipped objective and its five diagnostics in one pass.
//
// Drop-in signature tasks/ppo_clip/tests/task.json:3, replacing
// reference/ppo_clip/solution.cu:165-182.  The entropy variant adds TorchRL
// ClipPPOLoss's entropy bonus (mean entropy and -coef * mean entropy).  The kernel is in
// ppo_clip.hpp; the launch shape below is the measured best on MI355X.
#include "ppo_clip.hpp"

namespace taskops {
namespace {

constexpr int kThreads = 512;
constexpr int kUnroll = 2;
constexpr int kBlocksPerCU = 1;
constexpr bool kNonTemporal = true;

template <bool kEntropy>
hipError_t launch(int32_t B, int32_t T, int32_t H, const float* cur, const float* old,
                  const float* adv, const float* ent, float eps, float coef, float* out,
                  hipStream_t stream) {
  if (B <= 0 || T <= 0 || H <= 0) return hipErrorInvalidValue;
  const int64_t n = (int64_t)B * T * H;
  void* wsp = nullptr;
  hipError_t e = workspace(kSlotPpo, sizeof(PpoWorkspace), stream, &wsp);
  if (e != hipSuccess) return e;
  auto* ws = static_cast<PpoWorkspace*>(wsp);
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
                       dim3(kThreads), 0, stream, n, cur, old, adv, ent, p, coef, ws, out);
  else
    hipLaunchKernelGGL((ppo_clip_kernel<kThreads, kUnroll, false, kEntropy, kNonTemporal>), dim3(blocks),
                       dim3(kThreads), 0, stream, n, cur, old, adv, ent, p, coef, ws, out);
  return hipGetLastError();
}

}  // namespace
}  // namespace taskops

extern "C" hipError_t taskops_ppo_clip(int32_t B, int32_t T, int32_t H,
                                       const float* current_log_prob, const float* old_log_prob,
                                       const float* advantage, float clip_epsilon, float* output,
                                       hipStream_t stream) {
  return taskops::launch<false>(B, T, H, current_log_prob, old_log_prob, advantage, nullptr,
                                clip_epsilon, 0.0f, output, stream);
}

extern "C" hipError_t taskops_ppo_clip_entropy(int32_t B, int32_t T, int32_t H,
                                               const float* current_log_prob,
                                               const float* old_log_prob, const float* advantage,
                                               const float* entropy, float clip_epsilon,
                                               float entropy_coef, float* output,
                                               hipStream_t stream) {
  return taskops::launch<true>(B, T, H, current_log_prob, old_log_prob, advantage, entropy,
                               clip_epsilon, entropy_coef, output, stream);
}
