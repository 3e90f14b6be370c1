// Shared device helpers for the gfx950 task-op kernels: wave64 reductions, the
// agent-scope "last workgroup finishes" protocol, and the per-device cached workspace.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "taskops.h"

namespace taskops {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------
// Wave64 reductions.  XOR butterflies leave the result in every lane and fix the
// summation order, so the result is bitwise reproducible run to run.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Sum of one double per thread over a workgroup of kThreads threads.  The result is
// valid in every thread.  `lds` needs kThreads / 64 doubles.
template <int kThreads>
__device__ __forceinline__ double block_sum(double v, double* lds) {
  constexpr int kWaves = kThreads / kWave;
  v = wave_sum(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) t += lds[w];
  __syncthreads();
  return t;
}

// ---------------------------------------------------------------------------------------
// Single-launch grid reduction support.
//
// Every workgroup writes its partial record, then thread 0 takes a ticket with an
// agent-scope acq_rel atomic.  MI355X has 8 XCDs with private L2s: the release half
// writes the partial back past this XCD's L2 and the acquire half, taken by the last
// workgroup, invalidates stale lines before it reads the other XCDs' partials.  The
// last workgroup resets the ticket, so the next launch starts from zero.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ bool arrive_is_last(unsigned* ticket, bool* lds_flag) {
  __syncthreads();  // the whole workgroup's partial stores precede the ticket
  if (threadIdx.x == 0) {
    __threadfence();
    unsigned prev = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = (prev == gridDim.x - 1);
  }
  __syncthreads();
  bool last = *lds_flag;
  if (last) __threadfence();  // acquire for every thread of the finishing workgroup
  return last;
}

__device__ __forceinline__ void reset_ticket(unsigned* ticket) {
  __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ double load_coherent(const double* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------------------

// Workspace slots: one fixed-size region per op family, per device.
enum WorkspaceSlot : int {
  kSlotPow = 0,
  kSlotPpo = 1,
  kSlotKan = 2,
  kSlotFp8 = 3,
  kNumSlots = 4,
};

// Returns a zero-initialised device buffer of at least `bytes` for `slot` on the current
// device, allocated on the first request and kept until the process exits.  The zero
// fill is enqueued on `stream`, so it is ordered before the caller's first launch.
// A later request for more bytes than the first one returns hipErrorInvalidValue.
hipError_t workspace(WorkspaceSlot slot, size_t bytes, hipStream_t stream, void** out);

// Number of compute units of the current device (cached per device).
int device_cu_count();

}  // namespace taskops
