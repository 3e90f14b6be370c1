// fp8_linear on gfx950: output = bf16((x/sx) @ (w/sw)^T + bias), OCP e4m3 inputs.
//
// Drop-in signature tasks/fp8_linear/tests/task.json:3, replacing
// reference/fp8_linear/solution.cu:276-321.  Kernels are in fp8_linear.hpp: the skinny
// split-K kernel for M <= 64, the wide (direct-to-LDS, 128-byte rows) kernel when
// K % 16 == 0 and the operands are 16-byte aligned (in its 128-row form when 256x256
// tiles would fill at most half the CUs), and the register-staged tiled kernel otherwise.
#include "fp8_linear.hpp"

using namespace taskops;
using namespace taskops::fp8;

namespace {

// True when every 32-bit buffer offset of the kernels fits: a workgroup addresses its
// operand rows (at most 256 rows of K bytes above M = 64; all M rows of x and 16 of w in
// the skinny kernels) and, above M = 64, its output rows (at most 256 rows of N bf16
// values) through descriptors of at most 2^31 - 1 bytes.  The skinny grid (16 columns per
// workgroup of kSkinnyThreads) also stays within one launch's 2^32 - 1 work-items; above
// M = 64 the offsets bound N, which keeps that grid far inside it.
bool offsets_fit(int64_t M, int64_t K, int64_t N) {
  const int64_t lim = 0x7fffffff;
  if (M <= kSkinnyMaxM)
    return M * K <= lim && 16 * K <= lim && (N + 15) / 16 * kSkinnyThreads <= (int64_t)0xffffffff;
  return (int64_t)BM * K <= lim && (int64_t)BM * N * 2 <= lim;
}

}  // namespace

extern "C" hipError_t taskops_fp8_linear(int32_t M, int32_t K, int32_t N, const uint8_t* x_fp8,
                                         float scale_x, const uint8_t* w_fp8, float scale_w,
                                         const uint16_t* bias, uint16_t* output,
                                         hipStream_t stream) {
  if (M < 0 || K < 0 || N < 0) return hipErrorInvalidValue;
  if (M == 0 || N == 0) return hipSuccess;
  if (!offsets_fit(M, K, N)) return hipErrorInvalidValue;
  const float inv = (float)(1.0 / ((double)scale_x * (double)scale_w));
  const int vec = vec_width(x_fp8, w_fp8, K);
  if (M <= kSkinnyMaxM) {
    const dim3 grid((N + 15) / 16);
    if (vec == 16) {
      // Flat loads through LDS; M decides the row blocks (and so the K slice per pass).
      switch ((M + 15) / 16) {
        case 1:
          hipLaunchKernelGGL(fp8_gemm_skinny_flat<1>, grid, dim3(kSkinnyThreads), skinny_lds_bytes(1), stream,
                             x_fp8, w_fp8, (int)M, (int)N, (int)K, inv, bias, output);
          break;
        case 2:
          hipLaunchKernelGGL(fp8_gemm_skinny_flat<2>, grid, dim3(kSkinnyThreads), skinny_lds_bytes(2), stream,
                             x_fp8, w_fp8, (int)M, (int)N, (int)K, inv, bias, output);
          break;
        case 3:
          hipLaunchKernelGGL(fp8_gemm_skinny_flat<3>, grid, dim3(kSkinnyThreads), skinny_lds_bytes(3), stream,
                             x_fp8, w_fp8, (int)M, (int)N, (int)K, inv, bias, output);
          break;
        default:
          hipLaunchKernelGGL(fp8_gemm_skinny_flat<4>, grid, dim3(kSkinnyThreads), skinny_lds_bytes(4), stream,
                             x_fp8, w_fp8, (int)M, (int)N, (int)K, inv, bias, output);
          break;
      }
    } else if (vec == 8)
      hipLaunchKernelGGL(fp8_gemm_skinny<8>, grid, dim3(kSkinnyThreads), 0, stream, x_fp8, w_fp8,
                         (int)M, (int)N, (int)K, inv, bias, output);
    else
      hipLaunchKernelGGL(fp8_gemm_skinny<1>, grid, dim3(kSkinnyThreads), 0, stream, x_fp8, w_fp8,
                         (int)M, (int)N, (int)K, inv, bias, output);
    return hipGetLastError();
  }
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const size_t lds = 2 * kStageBytes;
  if (vec == 16) {
    const size_t wide_lds = kWideLdsBytes;
    const uintptr_t o = reinterpret_cast<uintptr_t>(output);
    if (2 * tiles <= device_cu_count()) {
      // At most half a 256x256 tile per CU: 128x256 tiles, twice as many workgroups.
      const dim3 hgrid(((M + kHalfRows - 1) / kHalfRows) * ((N + BN - 1) / BN));
      const size_t half_lds = kHalfLaunchLdsBytes;
      if (N % 8 == 0 && (o & 15) == 0)
        hipLaunchKernelGGL(fp8_gemm_half<2>, hgrid, dim3(kThreads), half_lds, stream, x_fp8, w_fp8, (int)M,
                           (int)N, (int)K, inv, bias, output);
      else if (N % 4 == 0 && (o & 7) == 0)
        hipLaunchKernelGGL(fp8_gemm_half<1>, hgrid, dim3(kThreads), half_lds, stream, x_fp8, w_fp8, (int)M,
                           (int)N, (int)K, inv, bias, output);
      else
        hipLaunchKernelGGL(fp8_gemm_half<0>, hgrid, dim3(kThreads), half_lds, stream, x_fp8, w_fp8, (int)M,
                           (int)N, (int)K, inv, bias, output);
      return hipGetLastError();
    }
    // K % 128 == 0: copies without per-lane bounds tests (copy_offset; the 128x256 form
    // measured no faster with them dropped).
    if (N % 8 == 0 && (o & 15) == 0 && K % WBK == 0)
      hipLaunchKernelGGL((fp8_gemm_wide<2, true>), dim3(tiles), dim3(kThreads), wide_lds, stream, x_fp8, w_fp8,
                         (int)M, (int)N, (int)K, inv, bias, output);
    else if (N % 8 == 0 && (o & 15) == 0)
      hipLaunchKernelGGL(fp8_gemm_wide<2>, dim3(tiles), dim3(kThreads), wide_lds, stream, x_fp8, w_fp8,
                         (int)M, (int)N, (int)K, inv, bias, output);
    else if (N % 4 == 0 && (o & 7) == 0)
      hipLaunchKernelGGL(fp8_gemm_wide<1>, dim3(tiles), dim3(kThreads), wide_lds, stream, x_fp8, w_fp8,
                         (int)M, (int)N, (int)K, inv, bias, output);
    else
      hipLaunchKernelGGL(fp8_gemm_wide<0>, dim3(tiles), dim3(kThreads), wide_lds, stream, x_fp8, w_fp8,
                         (int)M, (int)N, (int)K, inv, bias, output);
    return hipGetLastError();
  }
  if (vec == 8)
    hipLaunchKernelGGL(fp8_gemm_tiled<8>, dim3(tiles), dim3(kThreads), lds, stream, x_fp8, w_fp8,
                       (int)M, (int)N, (int)K, inv, bias, output);
  else
    hipLaunchKernelGGL(fp8_gemm_tiled<1>, dim3(tiles), dim3(kThreads), lds, stream, x_fp8, w_fp8,
                       (int)M, (int)N, (int)K, inv, bias, output);
  return hipGetLastError();
}
