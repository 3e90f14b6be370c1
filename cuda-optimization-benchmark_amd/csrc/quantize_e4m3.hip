// quantize_e4m3 on gfx950: per-tensor max-abs OCP e4m3 quantisation, the step that
// produces fp8_linear's operands.
//
// Op: tasks/fp8_linear/reference.py:15-18 (`_quantize`):
//   scale = fp32(448 / max(max|x|, 1e-9))      quotient in fp64 (a Python float), one rounding
//   q     = e4m3(clamp(x * scale, -448, 448))   fp32 product, round-to-nearest-even cast
// A NaN in x makes amax, scale and every q NaN: torch's max, Python's max(nan, 1e-9) and
// the casts all keep it.
//
// Two launches over x (HBM-bound).  qz_amax reduces |x| per workgroup as raw bits: for
// |x| the IEEE order is the unsigned-integer order and every NaN sorts above inf, so an
// integer max propagates NaN; each workgroup writes one partial.  qz_cast reduces those
// partials (every workgroup, a few KiB from L2), derives the scale, and converts 16
// values per thread with v_cvt_pk_fp8_f32 into one 16-byte store.  Algorithmic bytes are
// 4 in + 1 out per element; the second read of x is the price of the global max.
#include "common.hpp"

namespace taskops {
namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 16;  // elements per thread per grid-stride step
constexpr int kMaxPartials = 2048;
using f32x4 = float __attribute__((ext_vector_type(4)));
using u32x4 = unsigned __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned abs_bits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

__device__ __forceinline__ unsigned wave_max_u32(unsigned v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, (unsigned)__shfl_xor((int)v, off, kWave));
  return v;
}

// Max over the workgroup; valid in every thread.
__device__ __forceinline__ unsigned block_max_u32(unsigned v, unsigned* lds) {
  v = wave_max_u32(v);
  if (threadIdx.x % kWave == 0) lds[threadIdx.x / kWave] = v;
  __syncthreads();
  unsigned m = 0u;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) m = max(m, lds[w]);
  __syncthreads();
  return m;
}

template <bool kVec>
__global__ __launch_bounds__(kThreads) void qz_amax(const float* __restrict__ x, int64_t n,
                                                    unsigned* __restrict__ partial) {
  __shared__ unsigned lds[kThreads / kWave];
  unsigned m = 0u;
  const int64_t stride = (int64_t)gridDim.x * kThreads * kPerThread;
  for (int64_t i0 = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * kPerThread; i0 < n; i0 += stride) {
    if (kVec && i0 + kPerThread <= n) {
      const f32x4* p = reinterpret_cast<const f32x4*>(x + i0);
      f32x4 v[kPerThread / 4];
#pragma unroll
      for (int k = 0; k < kPerThread / 4; ++k) v[k] = __builtin_nontemporal_load(p + k);
#pragma unroll
      for (int k = 0; k < kPerThread / 4; ++k)
        m = max(max(m, max(abs_bits(v[k].x), abs_bits(v[k].y))), max(abs_bits(v[k].z), abs_bits(v[k].w)));
    } else {
      for (int64_t i = i0; i < i0 + kPerThread && i < n; ++i) m = max(m, abs_bits(x[i]));
    }
  }
  m = block_max_u32(m, lds);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// Two fp32 values to e4m3 bytes (round to nearest even) in bytes 0-1 (kHi false) or 2-3
// of `word`, the other half kept; the inputs are already within [-448, 448] or NaN.
template <bool kHi>
__device__ __forceinline__ unsigned cvt2(float a, float b, unsigned word) {
  return (unsigned)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)word, kHi);
}

// clamp(v * scale, -448, 448) with NaN kept (torch.clamp leaves NaN).
__device__ __forceinline__ float scaled(float v, float scale) {
  const float s = v * scale;
  return s < -448.0f ? -448.0f : (s > 448.0f ? 448.0f : s);
}

template <bool kVec>
__global__ __launch_bounds__(kThreads) void qz_cast(const float* __restrict__ x, int64_t n,
                                                    const unsigned* __restrict__ partial, int nparts,
                                                    uint8_t* __restrict__ q, float* __restrict__ scale_out) {
  __shared__ unsigned lds[kThreads / kWave];
  unsigned m = 0u;
  for (int i = threadIdx.x; i < nparts; i += kThreads) m = max(m, partial[i]);
  m = block_max_u32(m, lds);
  const float amax = __uint_as_float(m);
  // Python: max(amax, 1e-9) keeps a NaN amax; 448 / it in fp64, then np.float32.
  const double den = (m > 0x7F800000u) ? (double)amax : fmax((double)amax, 1e-9);
  const float scale = (float)(448.0 / den);
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;

  const int64_t stride = (int64_t)gridDim.x * kThreads * kPerThread;
  for (int64_t i0 = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * kPerThread; i0 < n; i0 += stride) {
    if (kVec && i0 + kPerThread <= n) {
      const f32x4* p = reinterpret_cast<const f32x4*>(x + i0);
      f32x4 v[kPerThread / 4];
#pragma unroll
      for (int k = 0; k < kPerThread / 4; ++k) v[k] = __builtin_nontemporal_load(p + k);
      u32x4 out;
#pragma unroll
      for (int k = 0; k < kPerThread / 4; ++k) {
        unsigned w = cvt2<false>(scaled(v[k].x, scale), scaled(v[k].y, scale), 0u);
        w = cvt2<true>(scaled(v[k].z, scale), scaled(v[k].w, scale), w);
        out[k] = w;
      }
      *reinterpret_cast<u32x4*>(q + i0) = out;
    } else {
      for (int64_t i = i0; i < i0 + kPerThread && i < n; ++i)
        q[i] = (uint8_t)(cvt2<false>(scaled(x[i], scale), 0.0f, 0u) & 0xFFu);
    }
  }
}

int grid_for(int64_t n, int per_cu) {
  const int64_t per_block = (int64_t)kThreads * kPerThread;
  int64_t g = (n + per_block - 1) / per_block;
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  if (g > cap) g = cap;
  if (g > kMaxPartials) g = kMaxPartials;
  return (int)(g < 1 ? 1 : g);
}

}  // namespace
}  // namespace taskops

using namespace taskops;

extern "C" hipError_t taskops_quantize_e4m3(const float* x, int64_t n, uint8_t* q, float* scale,
                                            hipStream_t stream) {
  if (n < 0) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;  // nothing to quantise; *scale is left as it is
  void* wsp = nullptr;
  hipError_t e = workspace(kSlotQuant, kMaxPartials * sizeof(unsigned), stream, &wsp);
  if (e != hipSuccess) return e;
  auto* partial = static_cast<unsigned*>(wsp);
  const bool vx = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  const bool vq = (reinterpret_cast<uintptr_t>(q) & 15) == 0;
  const int g1 = grid_for(n, 4);
  if (vx)
    hipLaunchKernelGGL((qz_amax<true>), dim3(g1), dim3(kThreads), 0, stream, x, n, partial);
  else
    hipLaunchKernelGGL((qz_amax<false>), dim3(g1), dim3(kThreads), 0, stream, x, n, partial);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int g2 = grid_for(n, 8);
  if (vx && vq)
    hipLaunchKernelGGL((qz_cast<true>), dim3(g2), dim3(kThreads), 0, stream, x, n, partial, g1, q, scale);
  else
    hipLaunchKernelGGL((qz_cast<false>), dim3(g2), dim3(kThreads), 0, stream, x, n, partial, g1, q, scale);
  return hipGetLastError();
}
