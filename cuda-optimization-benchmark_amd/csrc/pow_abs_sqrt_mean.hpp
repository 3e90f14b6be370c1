// pow_abs_sqrt_mean kernel template (instantiated by pow_abs_sqrt_mean.hip).
//
// Op: tasks/pow_abs_sqrt_mean/reference.py:22-28 (fp64 oracle :31-32).
// HBM-bound stream over two fp32 arrays (8 algorithmic bytes per element).  Each thread
// keeps kUnroll 16-byte loads of each input in flight per iteration (optionally
// non-temporal, so a 512 MiB stream does not churn the Infinity Cache), sums the
// 4*kUnroll terms of one iteration in fp32 and folds them into an fp64 accumulator.
// Workgroups reduce in fp64 and publish one double; the last workgroup to arrive sums
// the records in index order, so repeated calls give identical bits.
#pragma once

#include "common.hpp"

namespace taskops {

struct PowWorkspace {
  static constexpr int kMaxBlocks = 4096;
  double partial[kMaxBlocks];
  Arrivals arrivals;
};

namespace pow_detail {

using f32x4 = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float term(float a, float b) {
  const float d = a - b;
  return sqrtf(fmaf(d, d, 1.0e-6f));
}

__device__ __forceinline__ float term4(f32x4 a, f32x4 b) {
  return (term(a.x, b.x) + term(a.y, b.y)) + (term(a.z, b.z) + term(a.w, b.w));
}

template <bool kNT>
__device__ __forceinline__ f32x4 ld(const f32x4* p) {
  if constexpr (kNT) return __builtin_nontemporal_load(p);
  return *p;
}

}  // namespace pow_detail

template <int kThreads, int kUnroll, bool kVec, bool kNT>
__global__ __launch_bounds__(kThreads) void pow_abs_sqrt_mean_kernel(
    const float* __restrict__ a, const float* __restrict__ b, int64_t n,
    PowWorkspace* __restrict__ ws, float* __restrict__ out) {
  using namespace pow_detail;
  __shared__ double lds[kThreads / kWave];
  __shared__ bool last;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const int64_t tid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  double acc = 0.0;
  if constexpr (kVec) {
    const f32x4* a4 = reinterpret_cast<const f32x4*>(a);
    const f32x4* b4 = reinterpret_cast<const f32x4*>(b);
    const int64_t n4 = n >> 2;
    int64_t i = tid;
    for (; i + (kUnroll - 1) * stride < n4; i += kUnroll * stride) {
      f32x4 x[kUnroll], y[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        x[u] = ld<kNT>(a4 + i + u * stride);
        y[u] = ld<kNT>(b4 + i + u * stride);
      }
      float s = 0.0f;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) s += term4(x[u], y[u]);
      acc += (double)s;
    }
    for (; i < n4; i += stride) acc += (double)term4(ld<kNT>(a4 + i), ld<kNT>(b4 + i));
    if (tid < (n & 3)) {
      const int64_t k = (n4 << 2) + tid;
      acc += (double)term(a[k], b[k]);
    }
  } else {
    for (int64_t i = tid; i < n; i += stride) acc += (double)term(a[i], b[i]);
  }

  const double block = block_sum<kThreads>(acc, lds);
  if (!publish_and_arrive<1>(&ws->partial[blockIdx.x], &block, &ws->arrivals, &last)) return;
  double t = gather_records<false>(ws->partial, 1, (int)gridDim.x, threadIdx.x, kThreads);
  t = block_sum<kThreads>(t, lds);
  if (threadIdx.x == 0) {
    out[0] = (float)(t / (double)n);
  }
}

// Workgroups for n elements: enough to cover the work once, capped at kPerCU per CU.
inline int pow_grid(int64_t n, int threads, int unroll, bool vec, int cus, int per_cu) {
  const int64_t per_block = (int64_t)threads * unroll * (vec ? 4 : 1);
  int64_t blocks = (n + per_block - 1) / per_block;
  const int64_t cap = (int64_t)cus * per_cu;
  if (blocks > cap) blocks = cap;
  if (blocks > PowWorkspace::kMaxBlocks) blocks = PowWorkspace::kMaxBlocks;
  return blocks < 1 ? 1 : (int)blocks;
}

}  // namespace taskops
