// leaky kernel template (instantiated by leaky.hip).
//
// Op: tasks/leaky/reference.py:26-37 (the fp32 step loop is also the oracle, :40) and the
// step order of tasks/leaky/prompt.md.
//
// The recurrence is nonlinear (threshold reset), so time stays serial and the
// parallelism is over the B*H neurons.  A thread owns kVec adjacent neurons of one batch
// row and walks all T steps; step t reads x[t] (one 4*kVec-byte load, coalesced across
// the wave) and writes spikes[t].  Inputs are prefetched kDepth steps ahead in a register
// ring so each wave keeps kDepth loads in flight.  Arithmetic is fp32 with contraction
// disabled: each of beta*mem, +x, reset*th and the subtraction rounds once, exactly as
// the eager reference does, so spikes and final_mem are bit-identical to it.
// HBM-bound: 8 algorithmic bytes per neuron-step (4 in, 4 out).
#pragma once

#include "common.hpp"

#pragma clang fp contract(off)

namespace taskops {

namespace leaky_detail {
template <int kVec>
struct Vec;
template <>
struct Vec<1> {
  using T = float;
};
template <>
struct Vec<2> {
  using T = float __attribute__((ext_vector_type(2)));
};
template <>
struct Vec<4> {
  using T = float __attribute__((ext_vector_type(4)));
};

template <bool kNT, class V>
__device__ __forceinline__ V ld(const V* p) {
  if constexpr (kNT) return __builtin_nontemporal_load(p);
  return *p;
}
template <bool kNT, class V>
__device__ __forceinline__ void st(V v, V* p) {
  if constexpr (kNT)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}
}  // namespace leaky_detail

template <int kThreads, int kVec, int kDepth, bool kNT>
__global__ __launch_bounds__(kThreads) void leaky_kernel(
    const float* __restrict__ x, const float* __restrict__ mem0, const float* __restrict__ beta,
    const float* __restrict__ threshold, int T, int64_t N, int H, float* __restrict__ spikes,
    float* __restrict__ final_mem) {
  using namespace leaky_detail;
  using V = typename Vec<kVec>::T;
  const int64_t n0 = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * kVec;
  if (n0 >= N) return;
  const int h0 = (int)(n0 % H);

  float b[kVec], th[kVec], m[kVec];
#pragma unroll
  for (int k = 0; k < kVec; ++k) {
    float bb = beta[h0 + k];
    // clamp to [0, 1]; a NaN stays NaN, as torch.clamp leaves it
    bb = bb < 0.0f ? 0.0f : (bb > 1.0f ? 1.0f : bb);
    b[k] = bb;
    th[k] = threshold[h0 + k];
    m[k] = mem0[n0 + k];
  }

  const V* xp = reinterpret_cast<const V*>(x + n0);
  V* sp = reinterpret_cast<V*>(spikes + n0);
  const int64_t stride = N / kVec;  // one time step, in units of V

  V ring[kDepth];
#pragma unroll
  for (int j = 0; j < kDepth; ++j)
    if (j < T) ring[j] = ld<kNT>(xp + (int64_t)j * stride);

  for (int t0 = 0; t0 < T; t0 += kDepth) {
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      const int t = t0 + j;
      if (t >= T) break;
      const V xv = ring[j];
      if (t + kDepth < T) ring[j] = ld<kNT>(xp + (int64_t)(t + kDepth) * stride);
      V s;
      const float* xs = reinterpret_cast<const float*>(&xv);
      float* ss = reinterpret_cast<float*>(&s);
#pragma unroll
      for (int k = 0; k < kVec; ++k) {
        const float reset = (m[k] >= th[k]) ? 1.0f : 0.0f;
        const float decayed = b[k] * m[k];
        const float charged = decayed + xs[k];
        const float drop = reset * th[k];
        m[k] = charged - drop;
        ss[k] = (m[k] >= th[k]) ? 1.0f : 0.0f;
      }
      st<kNT>(s, sp + (int64_t)t * stride);
    }
  }
#pragma unroll
  for (int k = 0; k < kVec; ++k) final_mem[n0 + k] = m[k];
}

}  // namespace taskops
