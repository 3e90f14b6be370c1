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
// Single-launch grid reduction: publish a per-workgroup record, arrive, and let the last
// workgroup to arrive combine the records in a fixed order.
//
// MI355X has 8 XCDs with private L2s.  An agent-scope release (fence or acq_rel atomic)
// writes this XCD's whole L2 back; done by every workgroup it serialises per XCD and
// costs ~0.1 us per workgroup (measured: +190 us at 2048 workgroups).  Atomic RMWs at
// agent scope are instead performed at the device coherence point, so each workgroup
// publishes its record with agent-scope atomic exchanges, waits until they have
// returned, and only then arrives.  The last arrival reads the records with agent-scope
// atomic loads, which read the coherence point.
//
// Arrival is two-level.  RMWs on one address serialise at the coherence point (about
// 12 ns each: one counter cost 3.1 us at 256 workgroups), so workgroup b increments
// group counter b % kGroups, the group's last arrival increments the top counter, and
// the top counter's last arrival is the grid's last.  Each count is taken only after the
// previous RMW returned, so the chain orders every record exchange before the last
// arrival.  Counters are reset by the arrivals that finish them, so every launch leaves
// them zero (the workspace starts zeroed).
// ---------------------------------------------------------------------------------------
struct Arrivals {
  static constexpr int kGroups = 16;
  static constexpr int kSpacing = 16;  // one counter per 64-byte line
  unsigned c[(kGroups + 1) * kSpacing];
};

// Thread 0 publishes rec[0..n) into slot[0..n) and arrives; every thread of the
// workgroup learns whether it is the last to arrive.
template <int kN>
__device__ __forceinline__ bool publish_and_arrive(double* slot, const double* rec, Arrivals* arr,
                                                   bool* lds_flag) {
  if (threadIdx.x == 0) {
    unsigned long long seen = 0;
#pragma unroll
    for (int f = 0; f < kN; ++f) {
      seen |= __hip_atomic_exchange(reinterpret_cast<unsigned long long*>(slot) + f,
                                    __double_as_longlong(rec[f]), __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    }
    // Consume the exchanges' results so the arrival RMW issues only after they returned.
    asm volatile("" ::"v"(seen));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    constexpr unsigned kG = Arrivals::kGroups;
    const unsigned grid = gridDim.x, g = blockIdx.x % kG;
    const unsigned groups = grid < kG ? grid : kG;
    const unsigned members = grid / kG + (g < grid % kG ? 1u : 0u);
    unsigned* group = arr->c + g * Arrivals::kSpacing;
    unsigned* top = arr->c + kG * Arrivals::kSpacing;
    bool last = false;
    if (__hip_atomic_fetch_add(group, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == members - 1) {
      __hip_atomic_store(group, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == groups - 1) {
        __hip_atomic_store(top, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = true;
      }
    }
    *lds_flag = last;
  }
  __syncthreads();
  const bool last = *lds_flag;
  if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  return last;
}

__device__ __forceinline__ double load_coherent(const double* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The last workgroup's read of one field of the published records: base[j * stride] for
// j = first, first + step, ... < n, combined (sum, or max when kMax) in that order.  A
// coherent load is a round trip to the device coherence point (about 1.5 us), so loads go
// out kBatch at a time and their latencies overlap; one load per iteration would cost a
// round trip per record.  Records past n contribute 0 (the identity of the sums, and of
// the max over the non-negative values it is used for).
template <bool kMax, int kBatch = 8>
__device__ __forceinline__ double gather_records(const double* base, int stride, int n, int first, int step) {
  double t = 0.0;
  for (int j0 = first; j0 < n; j0 += kBatch * step) {
    double x[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int j = j0 + u * step;
      x[u] = j < n ? load_coherent(base + (int64_t)j * stride) : 0.0;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) t = kMax ? fmax(t, x[u]) : t + x[u];
  }
  return t;
}

// ---------------------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------------------

// Workspace slots: one fixed-size region per op family, per device.
enum WorkspaceSlot : int {
  kSlotPow = 0,
  kSlotPpo = 1,
  kSlotKan = 2,
  kSlotQuant = 3,
  kNumSlots = 4,
};

// Returns a zero-initialised device buffer of at least `bytes` for `slot` on the current
// device, allocated on the first request; hipErrorInvalidValue when `stream` belongs to
// another device.  A later request for more bytes allocates a
// larger one (the old one is kept until the process exits, since kernels enqueued before
// may still use it).  The zero fill is a kernel enqueued on `stream`, ordered before the
// caller's launches.
hipError_t workspace(WorkspaceSlot slot, size_t bytes, hipStream_t stream, void** out);

// Number of compute units of the current device (cached per device).
int device_cu_count();

// LDS bytes per compute unit of the current device (cached per device).
int device_lds_per_cu();

// Workgroup barrier without __syncthreads()'s release fence: that fence waits for every
// outstanding vector memory operation (vmcnt(0)), which would drain the copy ring at each
// step.  Callers account for their copies with explicit vmcnt waits; LDS reads issued
// before the barrier are complete (lgkmcnt(0)), and the signal fences keep the compiler
// from moving memory accesses across it.
__device__ __forceinline__ void barrier_no_vm_drain() {
  __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0x0 << 8) | 0xF | (0x3 << 14));  // lgkmcnt(0) only
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace taskops
