// pow_abs_sqrt_mean on gfx950: mean(sqrt((inp - target)^2 + 1e-6)) in one launch.
//
// Op: tasks/pow_abs_sqrt_mean/reference.py:22-28 (fp64 oracle :31-32); drop-in signature
// tasks/pow_abs_sqrt_mean/tests/task.json:3, replacing reference/pow_abs_sqrt_mean/solution.cu:99-118.
//
// HBM-bound stream over two fp32 arrays (8 algorithmic bytes per element).  Each thread
// keeps kUnroll 16-byte loads of each input in flight, sums the 4*kUnroll terms of one
// iteration in fp32 and folds them into an fp64 accumulator; workgroups reduce in fp64
// and the last workgroup to arrive (agent-scope ticket) sums the partials in a fixed
// order, so repeated calls give identical bits.
#include "common.hpp"

namespace taskops {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;
constexpr int kMaxBlocks = 4096;
constexpr int kBlocksPerCU = 8;

struct PowWorkspace {
  double partial[kMaxBlocks];
  unsigned ticket;
};

using f32x4 = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float term(float a, float b) {
  const float d = a - b;
  return sqrtf(fmaf(d, d, 1.0e-6f));
}

__device__ __forceinline__ float term4(f32x4 a, f32x4 b) {
  return (term(a.x, b.x) + term(a.y, b.y)) + (term(a.z, b.z) + term(a.w, b.w));
}

template <bool kVec>
__global__ __launch_bounds__(kThreads) void pow_abs_sqrt_mean_kernel(
    const float* __restrict__ a, const float* __restrict__ b, int64_t n,
    PowWorkspace* __restrict__ ws, float* __restrict__ out) {
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
        x[u] = a4[i + u * stride];
        y[u] = b4[i + u * stride];
      }
      float s = 0.0f;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) s += term4(x[u], y[u]);
      acc += (double)s;
    }
    for (; i < n4; i += stride) acc += (double)term4(a4[i], b4[i]);
    if (tid < (n & 3)) {
      const int64_t k = (n4 << 2) + tid;
      acc += (double)term(a[k], b[k]);
    }
  } else {
    for (int64_t i = tid; i < n; i += stride) acc += (double)term(a[i], b[i]);
  }

  const double block = block_sum<kThreads>(acc, lds);
  if (threadIdx.x == 0) ws->partial[blockIdx.x] = block;
  if (!arrive_is_last(&ws->ticket, &last)) return;
  double t = 0.0;
  for (int j = threadIdx.x; j < (int)gridDim.x; j += kThreads) t += load_coherent(&ws->partial[j]);
  t = block_sum<kThreads>(t, lds);
  if (threadIdx.x == 0) {
    out[0] = (float)(t / (double)n);
    reset_ticket(&ws->ticket);
  }
}

__global__ void write_nan_kernel(float* out) { out[0] = __builtin_nanf(""); }

}  // namespace
}  // namespace taskops

using namespace taskops;

extern "C" hipError_t taskops_pow_abs_sqrt_mean(const float* inp, const float* target,
                                                int64_t batch_size, int64_t height,
                                                int64_t width, float* output,
                                                hipStream_t stream) {
  if (batch_size < 0 || height < 0 || width < 0) return hipErrorInvalidValue;
  const int64_t n = batch_size * 4 * height * width;
  if (n == 0) {
    hipLaunchKernelGGL(write_nan_kernel, dim3(1), dim3(1), 0, stream, output);
    return hipGetLastError();
  }
  void* wsp = nullptr;
  hipError_t e = workspace(kSlotPow, sizeof(PowWorkspace), stream, &wsp);
  if (e != hipSuccess) return e;
  auto* ws = static_cast<PowWorkspace*>(wsp);
  const bool vec = ((reinterpret_cast<uintptr_t>(inp) | reinterpret_cast<uintptr_t>(target)) & 15) == 0;
  const int64_t per_block = (int64_t)kThreads * kUnroll * (vec ? 4 : 1);
  int64_t blocks = (n + per_block - 1) / per_block;
  const int64_t cap = (int64_t)device_cu_count() * kBlocksPerCU;
  if (blocks > cap) blocks = cap;
  if (blocks > kMaxBlocks) blocks = kMaxBlocks;
  if (blocks < 1) blocks = 1;
  if (vec)
    hipLaunchKernelGGL(pow_abs_sqrt_mean_kernel<true>, dim3((unsigned)blocks), dim3(kThreads), 0,
                       stream, inp, target, n, ws, output);
  else
    hipLaunchKernelGGL(pow_abs_sqrt_mean_kernel<false>, dim3((unsigned)blocks), dim3(kThreads), 0,
                       stream, inp, target, n, ws, output);
  return hipGetLastError();
}
