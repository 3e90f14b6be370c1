// fp8_linear on gfx950: output = bf16((x/sx) @ (w/sw)^T + bias), e4m3 inputs.
//
// Op: tasks/fp8_linear/reference.py:34-41 (fp64 oracle :44-45); drop-in signature
// tasks/fp8_linear/tests/task.json:3, replacing reference/fp8_linear/solution.cu:276-321.
//
// Scalar-FMA tiled version: 64x64 output tile per workgroup, e4m3 decoded into fp32 LDS
// tiles, fp32 accumulation, one round-to-nearest-even to bf16.
#include "common.hpp"

namespace taskops {
namespace {

constexpr int kTile = 64;
constexpr int kK = 32;

// OCP E4M3 (bias 7, no infinities, S.1111.111 is NaN) to fp32.
__device__ __forceinline__ float e4m3_to_f32(unsigned v) {
  const unsigned e = (v >> 3) & 15u, m = v & 7u;
  float mag;
  if (e == 15u && m == 7u) return __builtin_nanf("");
  if (e == 0u)
    mag = (float)m * 0x1p-9f;
  else
    mag = __builtin_ldexpf(1.0f + (float)m * 0.125f, (int)e - 7);
  return (v & 0x80u) ? -mag : mag;
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  unsigned u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__global__ __launch_bounds__(256) void fp8_linear_simple(int M, int K, int N, const uint8_t* __restrict__ x,
                                                         const uint8_t* __restrict__ w, float inv_scale,
                                                         const uint16_t* __restrict__ bias,
                                                         uint16_t* __restrict__ out) {
  __shared__ float xs[kK][kTile + 1];
  __shared__ float ws[kK][kTile + 1];
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const int m0 = blockIdx.y * kTile, n0 = blockIdx.x * kTile;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += kK) {
    for (int i = threadIdx.x; i < kTile * kK; i += 256) {
      const int r = i / kK, k = i % kK;
      const int gm = m0 + r, gn = n0 + r, gk = k0 + k;
      xs[k][r] = (gm < M && gk < K) ? e4m3_to_f32(x[(size_t)gm * K + gk]) : 0.0f;
      ws[k][r] = (gn < N && gk < K) ? e4m3_to_f32(w[(size_t)gn * K + gk]) : 0.0f;
    }
    __syncthreads();
    for (int k = 0; k < kK; ++k) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = xs[k][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = ws[k][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gm = m0 + ty + 16 * i, gn = n0 + tx + 16 * j;
      if (gm < M && gn < N) {
        const float bv = __uint_as_float((unsigned)bias[gn] << 16);
        out[(size_t)gm * N + gn] = f32_to_bf16_rne(acc[i][j] * inv_scale + bv);
      }
    }
}

}  // namespace
}  // namespace taskops

using namespace taskops;

extern "C" hipError_t taskops_fp8_linear(int32_t M, int32_t K, int32_t N, const uint8_t* x_fp8,
                                         float scale_x, const uint8_t* w_fp8, float scale_w,
                                         const uint16_t* bias, uint16_t* output,
                                         hipStream_t stream) {
  if (M < 0 || K < 0 || N < 0) return hipErrorInvalidValue;
  if (M == 0 || N == 0) return hipSuccess;
  const float inv = (float)(1.0 / ((double)scale_x * (double)scale_w));
  dim3 grid((N + kTile - 1) / kTile, (M + kTile - 1) / kTile);
  hipLaunchKernelGGL(fp8_linear_simple, grid, dim3(256), 0, stream, (int)M, (int)K, (int)N, x_fp8,
                     w_fp8, inv, bias, output);
  return hipGetLastError();
}
