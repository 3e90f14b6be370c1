// efficient_kan on gfx950: KANLinear forward.
//
// Op: tasks/efficient_kan/reference.py:33-51 (fp64 oracle :54-57); drop-in signature
// tasks/efficient_kan/tests/task.json:3, replacing reference/efficient_kan/solution.cu:177-288.
//
// Row-per-workgroup version: the expanded activation row [silu(x_i), B_0(x_i) ..
// B_{C-1}(x_i)] is built in LDS feature-chunk by feature-chunk with the Cox-de Boor
// recurrence, and each thread accumulates one output column in fp32.
#include "common.hpp"

namespace taskops {
namespace {

constexpr int kThreads = 256;
constexpr int kFeat = 128;     // features per LDS chunk
constexpr int kMaxKnots = 32;  // grid_size + 2*spline_order + 1
constexpr int kMaxC = kMaxKnots - 1;

// Cox-de Boor on one feature's knot row: order-0 indicators, then spline_order rounds.
__device__ void bsplines(const float* __restrict__ g, int L, int order, float x, float* out) {
  float b[kMaxKnots];
  for (int j = 0; j < L - 1; ++j) b[j] = (x >= g[j] && x < g[j + 1]) ? 1.0f : 0.0f;
  for (int k = 1; k <= order; ++k) {
    for (int j = 0; j < L - 1 - k; ++j) {
      const float left = (x - g[j]) / (g[j + k] - g[j]) * b[j];
      const float right = (g[j + k + 1] - x) / (g[j + k + 1] - g[j + 1]) * b[j + 1];
      b[j] = left + right;
    }
  }
  for (int c = 0; c < L - 1 - order; ++c) out[c] = b[c];
}

__global__ __launch_bounds__(kThreads) void kan_rowwise(
    const float* __restrict__ x, const float* __restrict__ grid, const float* __restrict__ wb,
    const float* __restrict__ ws, const float* __restrict__ sc, int G, int order, int I, int O,
    float* __restrict__ out) {
  extern __shared__ float lds[];  // [kFeat][1 + C]
  const int L = G + 2 * order + 1, C = G + order, S = 1 + C;
  const int b = blockIdx.y;
  const int o = blockIdx.x * kThreads + threadIdx.x;
  float acc = 0.0f;
  for (int i0 = 0; i0 < I; i0 += kFeat) {
    const int nf = min(kFeat, I - i0);
    __syncthreads();
    for (int f = threadIdx.x; f < nf; f += kThreads) {
      const float xv = x[(size_t)b * I + i0 + f];
      lds[f * S] = xv / (1.0f + expf(-xv));
      bsplines(grid + (size_t)(i0 + f) * L, L, order, xv, lds + f * S + 1);
    }
    __syncthreads();
    if (o < O) {
      for (int f = 0; f < nf; ++f) {
        const size_t oi = (size_t)o * I + i0 + f;
        float s = lds[f * S] * wb[oi];
        float t = 0.0f;
        for (int c = 0; c < C; ++c) t = fmaf(lds[f * S + 1 + c], ws[oi * C + c], t);
        acc += s + t * sc[oi];
      }
    }
  }
  if (o < O) out[(size_t)b * O + o] = acc;
}

}  // namespace
}  // namespace taskops

using namespace taskops;

extern "C" hipError_t taskops_efficient_kan(const float* x, const float* grid,
                                            const float* base_weight, const float* spline_weight,
                                            const float* spline_scaler, int32_t grid_size,
                                            int32_t spline_order, int32_t B, int32_t I, int32_t O,
                                            float* out, hipStream_t stream) {
  if (B < 0 || I < 0 || O < 0 || grid_size < 1 || spline_order < 0) return hipErrorInvalidValue;
  if (grid_size + 2 * spline_order + 1 > kMaxKnots) return hipErrorInvalidValue;
  if (B == 0 || O == 0) return hipSuccess;
  const int S = 1 + grid_size + spline_order;
  dim3 g((O + kThreads - 1) / kThreads, B);
  hipLaunchKernelGGL(kan_rowwise, g, dim3(kThreads), (size_t)kFeat * S * sizeof(float), stream, x,
                     grid, base_weight, spline_weight, spline_scaler, (int)grid_size,
                     (int)spline_order, (int)I, (int)O, out);
  return hipGetLastError();
}
