// reward_to_go on gfx950: batched discounted reward-to-go with done flags.
//
// Op: tasks/reward_to_go/reference.py:34-42 (fp64 backward loop); prompt text
// tasks/reward_to_go/prompt.md ("output[b,t] = reward[b,t] + gamma * next");
// drop-in signature tasks/reward_to_go/tests/task.json:3, replacing
// reference/reward_to_go/solution.cu:237-264.
//
// Each time step is the affine map  v -> r[t] + a[t] * v  with a[t] = done[t] ? 0 : gamma,
// and out[t] is the composition of the maps t..T-1 applied to 0.  One wave64 owns one
// row.  The row is cut into chunks of 256 steps (4 per lane, loaded as one 16-byte reward
// vector and one 4-byte done word per lane, so every load instruction covers 1 KiB of
// contiguous reward).  Per chunk, each lane composes its 4 maps, the wave runs a
// log-depth suffix scan of the lane maps (6 shuffle steps), and the value flowing in from
// the later chunk (the carry) is applied.  Chunks are processed from the row end toward
// its start; kSeg chunks are loaded up front (10 KiB in flight per wave at 110 VGPRs, so 4 waves
// per SIMD hold a 4096-row batch resident at once).  The
// maps and the carry are fp64, and each output is rounded to fp32 once.
// HBM-bound: 9 algorithmic bytes per element (4 reward + 1 done + 4 out).
#include "common.hpp"

namespace taskops {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kThreads = kWavesPerBlock * kWave;
constexpr int kPerLane = 4;
constexpr int kChunk = kWave * kPerLane;
constexpr int kSeg = 8;

template <bool kVec>
__global__ __launch_bounds__(kThreads) void reward_to_go_kernel(
    const float* __restrict__ reward, const uint8_t* __restrict__ done, double g, int B, int T,
    float* __restrict__ out) {
  const int lane = threadIdx.x % kWave;
  const int row = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (row >= B) return;  // whole wave leaves; no workgroup barrier below
  const size_t base = (size_t)row * (size_t)T;
  const float* rr = reward + base;
  const uint8_t* dd = done + base;
  float* oo = out + base;
  const int nchunks = (T + kChunk - 1) / kChunk;

  double carry = 0.0;  // value of the step after the current chunk (0 past the row end)
  for (int hi = nchunks; hi > 0; hi -= kSeg) {
    const int lo = hi > kSeg ? hi - kSeg : 0;
    float r[kSeg][kPerLane];
    unsigned dn[kSeg];
#pragma unroll
    for (int c = 0; c < kSeg; ++c) {
      const int t0 = (lo + c) * kChunk + lane * kPerLane;
      dn[c] = 0u;
#pragma unroll
      for (int e = 0; e < kPerLane; ++e) r[c][e] = 0.0f;
      if (lo + c >= hi) continue;
      if constexpr (kVec) {
        if (t0 < T) {
          const float4 v = *reinterpret_cast<const float4*>(rr + t0);
          r[c][0] = v.x;
          r[c][1] = v.y;
          r[c][2] = v.z;
          r[c][3] = v.w;
          dn[c] = *reinterpret_cast<const unsigned*>(dd + t0);
        }
      } else {
#pragma unroll
        for (int e = 0; e < kPerLane; ++e) {
          if (t0 + e < T) {
            r[c][e] = rr[t0 + e];
            dn[c] |= (unsigned)(dd[t0 + e] != 0) << (8 * e);
          }
        }
      }
    }

#pragma unroll
    for (int c = kSeg - 1; c >= 0; --c) {
      if (lo + c >= hi) continue;
      const int t0 = (lo + c) * kChunk + lane * kPerLane;
      double a[kPerLane];
#pragma unroll
      for (int e = 0; e < kPerLane; ++e) a[e] = ((dn[c] >> (8 * e)) & 0xFFu) ? 0.0 : g;
      // This lane's map over its 4 steps: v -> R + A * v.
      double R = 0.0, A = 1.0;
#pragma unroll
      for (int e = kPerLane - 1; e >= 0; --e) {
        R = fma(a[e], R, (double)r[c][e]);
        A = a[e] * A;
      }
      // Suffix scan: lane l ends with the map of lanes l..63 of this chunk.
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const double Rn = __shfl_down(R, off, kWave);
        const double An = __shfl_down(A, off, kWave);
        if (lane + off < kWave) {
          R = fma(A, Rn, R);
          A = A * An;
        }
      }
      // Value after this lane's steps: the later lanes' map applied to the carry.
      const double Rn = __shfl_down(R, 1, kWave);
      const double An = __shfl_down(A, 1, kWave);
      double v = (lane == kWave - 1) ? carry : fma(An, carry, Rn);
      float o[kPerLane];
#pragma unroll
      for (int e = kPerLane - 1; e >= 0; --e) {
        v = fma(a[e], v, (double)r[c][e]);
        o[e] = (float)v;
      }
      if constexpr (kVec) {
        if (t0 < T) *reinterpret_cast<float4*>(oo + t0) = make_float4(o[0], o[1], o[2], o[3]);
      } else {
#pragma unroll
        for (int e = 0; e < kPerLane; ++e)
          if (t0 + e < T) oo[t0 + e] = o[e];
      }
      carry = __shfl(v, 0, kWave);  // value at the chunk's first step
    }
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
  const bool vec = (T % kPerLane) == 0 &&
                   ((reinterpret_cast<uintptr_t>(reward) | reinterpret_cast<uintptr_t>(output)) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(d) & 3) == 0;
  const unsigned blocks = (unsigned)((B + kWavesPerBlock - 1) / kWavesPerBlock);
  const double g = (double)gamma;
  if (vec)
    hipLaunchKernelGGL(reward_to_go_kernel<true>, dim3(blocks), dim3(kThreads), 0, stream, reward, d,
                       g, (int)B, (int)T, output);
  else
    hipLaunchKernelGGL(reward_to_go_kernel<false>, dim3(blocks), dim3(kThreads), 0, stream, reward,
                       d, g, (int)B, (int)T, output);
  return hipGetLastError();
}
