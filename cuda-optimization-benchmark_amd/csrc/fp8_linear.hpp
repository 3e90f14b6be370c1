// fp8_linear kernels for gfx950 (instantiated by fp8_linear.hip):
// output = bf16((x/sx) @ (w/sw)^T + bias), OCP e4m3 inputs.
//
// Op: tasks/fp8_linear/reference.py:34-41 (fp64 oracle :44-45, one rounding to bf16);
// drop-in signature tasks/fp8_linear/tests/task.json:3, replacing
// reference/fp8_linear/solution.cu:276-321 (there: dequantise + cuBLASLt).
//
// Both operands are K-contiguous e4m3 ([M,K] and [N,K]), which is exactly the operand
// layout of gfx950's scaled MFMA v_mfma_scale_f32_16x16x128_f8f6f4 (format 0 = e4m3,
// block scales set to 2^0): lane l supplies 32 consecutive k of row (l % 16) starting at
// k = 32*(l / 16), for A and B alike, and gets back D rows 4*(l/16)..+3 of column l % 16.
// The product is accumulated in fp32 and the epilogue applies 1/(sx*sw), adds the bf16
// bias and rounds to bf16 (nearest-even) once.
//
// Three kernels, one launch per call:
//  * wide (M > 64, K % 16 == 0, 16-byte aligned operands): the main path, described at
//    fp8_gemm_wide below — direct-to-LDS copies of whole 128-byte row segments into two
//    64 KiB stages, 32x32x64 MFMAs with fragments read a half-step ahead.  Grids of at
//    most half a 256x256 tile per CU take its 128x256-tile form, fp8_gemm_half.
//  * tiled (M > 64, other K or alignment): 256x256 output tile per workgroup of 4 waves (one per SIMD, each
//    128x128 = 8x8 MFMA blocks whose 256 fp32 accumulators sit in AGPRs), K in steps of
//    128 staged through LDS (2 stages x 64 KiB, 16-byte
//    chunks XOR-swizzled by row so a wave's fragment reads spread over the banks).  The
//    next K-step's global loads are in flight while the current one feeds the MFMAs.
//    Workgroups are mapped so that each XCD's 32 concurrent tiles form a 4x8 block of
//    the output and share A/B panels in that XCD's L2.
//  * skinny (M <= 64): the weight-streaming case.  A workgroup owns 16 output columns
//    and all M rows; its 8 waves split K, read W straight from global memory into MFMA
//    fragments, and reduce their partial tiles through LDS in a fixed order.
#pragma once

#include "common.hpp"

namespace taskops {
namespace fp8 {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kScaleOne = 0x7f7f7f7f;  // E8M0 127 in every byte: 2^0

__device__ __forceinline__ f32x4 mfma_e4m3(i32x8 a, i32x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, kScaleOne, 0, kScaleOne);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  unsigned u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((unsigned)b << 16); }

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats to two bf16 (round to nearest even) packed low-first: one
// v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ unsigned pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// Buffer resources: a 128-bit descriptor (base, byte size) makes the hardware return zero
// for loads past the size and drop stores past it, so tile tails need no branches.
// Offsets are 32-bit, so each workgroup bases its descriptors at its own tile.
constexpr int kRawBufferFlags = 0x00020000;  // raw (untyped) 32-bit buffer, gfx9 layout
constexpr unsigned kOutOfRange = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, size_t bytes) {
  const int n = bytes > 0x7fffffffu ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, kRawBufferFlags);
}

// 16 bytes of a K-contiguous row starting at column k, zero past K.  `off` is the byte
// offset of (row, k) in the descriptor, or kOutOfRange for rows past the matrix.
// kVec 16: K % 16 == 0, a chunk is wholly inside or outside K; 8: K % 8 == 0, two
// independent halves; 1: any K, byte by byte.
template <int kVec>
__device__ __forceinline__ i32x4 load16(__amdgpu_buffer_rsrc_t r, unsigned off, int k, int K) {
  if constexpr (kVec == 16) {
    const unsigned o = k < K ? off : kOutOfRange;
    return __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0));
  } else if constexpr (kVec == 8) {
    const unsigned o0 = k < K ? off : kOutOfRange;
    const unsigned o1 = k + 8 < K ? off + 8 : kOutOfRange;
    const i32x2 lo = __builtin_bit_cast(i32x2, __builtin_amdgcn_raw_buffer_load_b64(r, o0, 0, 0));
    const i32x2 hi = __builtin_bit_cast(i32x2, __builtin_amdgcn_raw_buffer_load_b64(r, o1, 0, 0));
    return i32x4{lo.x, lo.y, hi.x, hi.y};
  } else {
    unsigned w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const unsigned o = (k + i < K && off != kOutOfRange) ? off + i : kOutOfRange;
      w[i / 4] |= (unsigned)__builtin_amdgcn_raw_buffer_load_b8(r, o, 0, 0) << (8 * (i % 4));
    }
    return i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
}

__device__ __forceinline__ i32x8 join(i32x4 a, i32x4 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// ---------------------------------------------------------------------------------------
// Tiled kernel
// ---------------------------------------------------------------------------------------
constexpr int BM = 256, BN = 256, BK = 128;
constexpr int kThreads = 256;
constexpr int kWavesN = 2;                       // waves arranged 2 (M) x 2 (N)
constexpr int WM = 128, WN = 128;                // wave tile
constexpr int kMI = WM / 16, kNJ = WN / 16;      // 16x16 MFMA blocks per wave tile
constexpr int kStageBytes = (BM + BN) * BK;  // 64 KiB: A tile then B tile
constexpr int kChunksPerRow = BK / 16;       // 8
constexpr int kLoadsPerThread = BM * kChunksPerRow / kThreads;  // 16-byte chunks per operand

__device__ __forceinline__ int swizzle(int row, int chunk) {
  return row * BK + ((chunk ^ (row & 7)) << 4);
}

// Output tile of workgroup `b` (a bijection onto the tm x tn tiles for any tile counts).
// Workgroups are dispatched to the 8 XCDs round-robin (b % 8), so when the tile count is
// a multiple of 8, XCD x is given the contiguous run of virtual tiles
// [x*T/8, (x+1)*T/8); virtual tiles are then laid out in groups of kGroupM tile rows,
// column by column, so a run of 32 forms a 4x8 block whose A and B panels stay in that
// XCD's L2.
constexpr int kGroupM = 4;
__device__ __forceinline__ void tile_of(int b, int tm, int tn, int& mt, int& nt) {
  const int T = tm * tn;
  const int v = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
  const int per_group = kGroupM * tn;
  const int first_m = (v / per_group) * kGroupM;
  const int rows = min(tm - first_m, kGroupM);
  const int r = v % per_group;
  mt = first_m + r % rows;
  nt = r / rows;
}

template <int kVec>
__global__ __launch_bounds__(kThreads) void fp8_gemm_tiled(
    const uint8_t* __restrict__ x, const uint8_t* __restrict__ w, int M, int N, int K,
    float inv_scale, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  int mt, nt;
  tile_of(blockIdx.x, tm, tn, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int wm = wave / kWavesN, wn = wave % kWavesN;  // wave tile origin (wm*WM, wn*WN)
  const int rows_a = min(BM, M - m0), rows_b = min(BN, N - n0);
  const __amdgpu_buffer_rsrc_t xa = make_rsrc(x + (size_t)m0 * K, (size_t)rows_a * K);
  const __amdgpu_buffer_rsrc_t wb = make_rsrc(w + (size_t)n0 * K, (size_t)rows_b * K);

  i32x4 ra[kLoadsPerThread], rb[kLoadsPerThread];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i) {
      const int q = tid + kThreads * i;
      const int row = q / kChunksPerRow, chunk = q % kChunksPerRow;
      const int gk = k0 + chunk * 16;
      const unsigned off = (unsigned)(row * K + gk);
      ra[i] = load16<kVec>(xa, row < rows_a ? off : kOutOfRange, gk, K);
      rb[i] = load16<kVec>(wb, row < rows_b ? off : kOutOfRange, gk, K);
    }
  };
  auto swrite = [&](int stage) {
    uint8_t* As = smem + stage * kStageBytes;
    uint8_t* Bs = As + BM * BK;
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i) {
      const int q = tid + kThreads * i;
      const int row = q / kChunksPerRow, chunk = q % kChunksPerRow;
      *reinterpret_cast<i32x4*>(As + swizzle(row, chunk)) = ra[i];
      *reinterpret_cast<i32x4*>(Bs + swizzle(row, chunk)) = rb[i];
    }
  };

  f32x4 acc[kMI][kNJ];
#pragma unroll
  for (int i = 0; i < kMI; ++i)
#pragma unroll
    for (int j = 0; j < kNJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (K + BK - 1) / BK;
  gload(0);
  swrite(0);
  __syncthreads();
  const int fr = lane % 16, fg = lane / 16;  // fragment row and k-group of this lane
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
    const uint8_t* As = smem + cur * kStageBytes;
    const uint8_t* Bs = As + BM * BK;
    i32x8 bf[kNJ];
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
      const int row = wn * WN + j * 16 + fr;
      bf[j] = join(*reinterpret_cast<const i32x4*>(Bs + swizzle(row, 2 * fg)),
                   *reinterpret_cast<const i32x4*>(Bs + swizzle(row, 2 * fg + 1)));
    }
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
      const int row = wm * WM + i * 16 + fr;
      const i32x8 af = join(*reinterpret_cast<const i32x4*>(As + swizzle(row, 2 * fg)),
                            *reinterpret_cast<const i32x4*>(As + swizzle(row, 2 * fg + 1)));
#pragma unroll
      for (int j = 0; j < kNJ; ++j) acc[i][j] = mfma_e4m3(af, bf[j], acc[i][j]);
    }
    if (kt + 1 < nk) swrite(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds rows 4*fg..4*fg+3 of column fr in every 16x16 block.  Stores go
  // through a descriptor covering this tile's rows; columns past N get an out-of-range
  // offset and are dropped.
  // All bias loads are issued before the first store: vmcnt also counts stores, so a load
  // between stores would wait for every earlier store to complete.
  const __amdgpu_buffer_rsrc_t ob = make_rsrc(out + (size_t)m0 * N, (size_t)rows_a * N * 2);
  float bvs[kNJ];
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    const int gn = n0 + wn * WN + j * 16 + fr;
    bvs[j] = gn < N ? bf16_to_f32(bias[gn]) : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    const int gn = n0 + wn * WN + j * 16 + fr;
    const float bv = bvs[j];
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = wm * WM + i * 16 + 4 * fg + r;
        const unsigned off = gn < N ? (unsigned)(row * N + gn) * 2u : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_rne(acc[i][j][r] * inv_scale + bv), ob, off, 0, 0);
      }
    }
  }
}

constexpr int kSlotsPerInst = 64;  // a direct-to-LDS instruction writes 64 x 16 bytes

// ---------------------------------------------------------------------------------------
// Shared pieces of the wide kernel: 32x32x64 MFMA, vmcnt waits, epilogues, bias staging.
// ---------------------------------------------------------------------------------------
typedef float f32x16 __attribute__((ext_vector_type(16)));

// v_mfma_scale_f32_32x32x64_f8f6f4: lane l supplies 32 consecutive k of row l % 32
// starting at k = 32*(l/32); D register r of lane l is row 8*(r/4) + 4*(l/32) + r%4,
// column l % 32.
__device__ __forceinline__ f32x16 mfma32_e4m3(i32x8 a, i32x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, kScaleOne, 0, kScaleOne);
}

// s_waitcnt with vmcnt <= n and the other counters unconstrained (gfx9 encoding).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Direct epilogue of the wide kernel.  acc[i][j] is the transposed 32x32 block (output rows
// i*32.., columns j*32.. of this wave's tile): lane l holds output row l % 32 and, in
// registers 4q..4q+3, columns 8q + 4*(l/32) + 0..3.  With kVec4 (N % 4 == 0) those four
// columns go out as one 8-byte store; otherwise one 2-byte store each.  Columns past N
// get an out-of-range offset and are dropped by the buffer descriptor.  bias_s holds the
// tile's BN bias values in LDS (zero past N), so no global load sits between the stores.
// kMIx: 32-row x blocks per wave (4 in the 256-row tile, 2 in the 128-row one).
template <bool kVec4, int kMIx = 4>
__device__ __forceinline__ void store_transposed_block(const f32x16 (&acc)[kMIx][4], uint16_t* out,
                                                       const uint16_t* bias_s, int N, int m0,
                                                       int n0, int wm, int wn, int fr, int fg,
                                                       int rows_a, float inv_scale) {
  const __amdgpu_buffer_rsrc_t ob = make_rsrc(out + (size_t)m0 * N, (size_t)rows_a * N * 2);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = wn * WN + j * 32 + 8 * q + 4 * fg;  // first of four tile columns
      const int gn = n0 + c;
      const i32x2 braw = *reinterpret_cast<const i32x2*>(bias_s + c);
      const float bv[4] = {__uint_as_float((unsigned)braw.x << 16), __uint_as_float((unsigned)braw.x & 0xffff0000u),
                           __uint_as_float((unsigned)braw.y << 16), __uint_as_float((unsigned)braw.y & 0xffff0000u)};
#pragma unroll
      for (int i = 0; i < kMIx; ++i) {
        const int row = wm * 32 * kMIx + i * 32 + fr;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = fmaf(acc[i][j][4 * q + e], inv_scale, bv[e]);
        const unsigned p01 = pack_bf16x2(v[0], v[1]), p23 = pack_bf16x2(v[2], v[3]);
        if constexpr (kVec4) {
          const unsigned off = gn < N ? (unsigned)(row * N + gn) * 2u : kOutOfRange;
          typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
          __builtin_amdgcn_raw_buffer_store_b64(u32x2{p01, p23}, ob, off, 0, 0);
        } else {
          const unsigned short h[4] = {(unsigned short)p01, (unsigned short)(p01 >> 16),
                                       (unsigned short)p23, (unsigned short)(p23 >> 16)};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const unsigned off = gn + e < N ? (unsigned)(row * N + gn + e) * 2u : kOutOfRange;
            __builtin_amdgcn_raw_buffer_store_b16(h[e], ob, off, 0, 0);
          }
        }
      }
    }
  }
}

// Epilogue through LDS (N % 8 == 0, 16-byte aligned output): the 256x256 (or 128x256)
// bf16 tile is assembled in `tile_s` (128 or 64 KiB of the rings, once every copy has
// landed and every wave is past its last fragment read), then each store instruction writes two whole
// 512-byte tile rows, instead of 16 bytes into each of 32 rows.  Tile row r's 16-byte
// chunk c sits at chunk c ^ (r % 32), so both the column-wise writes and the row-wise
// reads spread over all banks.
constexpr int kTileRowBytes = BN * 2;  // 512
constexpr int kCachePolicyNT = 2;       // buffer load/store cache-policy operand: nt
template <int kMIx = 4>  // 32-row x blocks per wave: the tile has 64 * kMIx rows
__device__ __forceinline__ void store_tile_lds(const f32x16 (&acc)[kMIx][4], uint16_t* out,
                                               const uint16_t* bias_s, uint8_t* tile_s, int N,
                                               int m0, int n0, int wm, int wn, int fr, int fg,
                                               int rows_a, int rows_b, float inv_scale, int tid) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = wn * WN + j * 32 + 8 * q + 4 * fg;  // first of four tile columns
      const i32x2 braw = *reinterpret_cast<const i32x2*>(bias_s + c);
      const float bv[4] = {__uint_as_float((unsigned)braw.x << 16), __uint_as_float((unsigned)braw.x & 0xffff0000u),
                           __uint_as_float((unsigned)braw.y << 16), __uint_as_float((unsigned)braw.y & 0xffff0000u)};
#pragma unroll
      for (int i = 0; i < kMIx; ++i) {
        const int r = wm * 32 * kMIx + i * 32 + fr;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = fmaf(acc[i][j][4 * q + e], inv_scale, bv[e]);
        const int chunk = c / 8, half = (c / 4) & 1;
        *reinterpret_cast<i32x2*>(tile_s + r * kTileRowBytes + ((chunk ^ (r & 31)) << 4) + 8 * half) =
            i32x2{(int)pack_bf16x2(v[0], v[1]), (int)pack_bf16x2(v[2], v[3])};
      }
    }
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t ob = make_rsrc(out + (size_t)m0 * N, (size_t)rows_a * N * 2);
  const int lane = tid % kWave, wave = tid / kWave;
  const int chunk = lane % 32;
  const bool col_ok = chunk * 8 < rows_b;  // rows_b: valid columns of this tile (N % 8 == 0)
#pragma unroll 4
  for (int s = 0; s < 64 * kMIx / 2 / (kThreads / kWave); ++s) {
    const int r = (wave * (64 * kMIx / 2 / (kThreads / kWave)) + s) * 2 + lane / 32;
    const i32x4 v = *reinterpret_cast<const i32x4*>(tile_s + r * kTileRowBytes + ((chunk ^ (r & 31)) << 4));
    const unsigned off = (r < rows_a && col_ok) ? (unsigned)(r * N + n0 + chunk * 8) * 2u : kOutOfRange;
    // Non-temporal (streaming) stores: the 32 MB output of a 4096^2 call otherwise sits dirty
    // in L2 and is written back after the last workgroup ends, adding ~3 us per call.
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v), ob, off, 0,
                                           kCachePolicyNT);
  }
}

// Bias staging for the wide kernel: thread t (kThreads == BN) loads bias[n0 + t] (zero
// past N); the kernel writes it to LDS past the output tile, where the epilogue reads it.
static_assert(kThreads == BN, "one bias value per thread");
static_assert(BM * kTileRowBytes + BN * 2 <= 5 * BM * 128, "the output tile and bias fit the LDS rings");
constexpr int kBiasBytes = BN * 2;
__device__ __forceinline__ unsigned short load_bias(const uint16_t* bias, int n0, int rows_b, int tid) {
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(bias + n0, (size_t)rows_b * 2);
  return __builtin_amdgcn_raw_buffer_load_b16(rb, tid < rows_b ? (unsigned)tid * 2u : kOutOfRange, 0, 0);
}


// ---------------------------------------------------------------------------------------
// Wide kernel (the main path: M > 64, K % 16 == 0, 16-byte aligned operands).
//
// 256x256 output tile, 4 waves of 128x128 (4x4 blocks of 32x32x64 MFMAs, accumulators in
// AGPRs), W fed as the A operand so D is the transposed block.  The copy engine's rate is
// set by requests, not bytes: measured on MI355X, a 128-byte run per row moves ~45% more
// per clock than a 64-byte one.  So K advances in steps of 128 (each tile row is one whole
// 128-byte line), each operand's 32 KiB per step through its own LDS ring: x (A) has three
// slots, w (B) two, 160 KiB in all.  Each step is two halves of 64 k (16 MFMAs per wave
// each); the fragments of the second half are read while the first half's MFMAs run, and
// those of the next step's first half while the second half's run.  A copy instruction
// moves 1 KiB and the memory pipeline takes about one per MFMA from the four waves
// together, so issuing more at once stalls the MFMAs behind them: step kt+2's x copies go
// out during step kt's first half, into the slot step kt-1 left (every wave passed the
// barrier at its mid-step), and its w copies during the second half, into the slot step kt
// left at this mid-step; one copy per two MFMAs throughout.  Row r's 16-byte chunk c sits
// at chunk c ^ ((r >> 1) & 7), which spreads any 16 consecutive rows of one chunk over all
// banks.  Accumulation order is k ascending in 64-wide MFMA steps, as in the tiled
// kernel's 128-wide steps of two 64-wide halves.
// ---------------------------------------------------------------------------------------
constexpr int WBK = 128;
constexpr int kWideOperandBytes = BM * WBK;                          // 32 KiB per operand and step
constexpr int kWideLdsBytes = 5 * kWideOperandBytes;                 // 3 x-slots + 2 w-slots: 160 KiB
static_assert(BM == BN, "both operands' slots hold 256 rows");
constexpr int kWideDmaPerWave = (BM * WBK / 16) / kSlotsPerInst / (kThreads / kWave);  // 8

__device__ __forceinline__ int swz128(int row) { return (row >> 1) & 7; }

// Byte offset of (row, gk) in a tile's descriptor for a 16-byte copy, or kOutOfRange.  With
// kK128 (K % 128 == 0) a step never straddles K, so no per-lane test is needed: rows past the
// tile lie past the descriptor's end and read zeros, and a step wholly past K only fills a
// slot that no MFMA uses (its offsets stay below 256 K + 384, inside 32 bits).
template <bool kK128>
__device__ __forceinline__ unsigned copy_offset(int row, int rows, int gk, int K) {
  const unsigned off = (unsigned)row * (unsigned)K + (unsigned)gk;
  if constexpr (kK128) return off;
  return (row < rows && gk < K) ? off : kOutOfRange;
}

// This wave's 8-row groups i0 .. i0+n-1 of a 256-row tile with 128-byte rows.
template <bool kK128>
__device__ __forceinline__ void dma_tile128(__amdgpu_buffer_rsrc_t r, uint8_t* lds_tile, int rows,
                                            int K, int k0, int wave, int lane, int i0 = 0,
                                            int n = kWideDmaPerWave) {
  const int r8 = lane / 8, p = lane % 8;  // row within the 8-row group, physical chunk
#pragma unroll
  for (int i = i0; i < i0 + n; ++i) {
    const int group = wave * kWideDmaPerWave + i;  // 8 rows per instruction
    const int row = group * 8 + r8;
    const int gk = k0 + 16 * (p ^ swz128(row));
    const unsigned off = copy_offset<kK128>(row, rows, gk, K);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)(lds_tile + group * kSlotsPerInst * 16), 16, off,
        0, 0, 0);
  }
}

// 16 bytes (part 0 or 1) of row `row` at k = 64*half + 32*fg + 16*part of a 128-byte-row tile.
__device__ __forceinline__ i32x4 frag128_part(const uint8_t* tile, int row, int fg, int half, int part) {
  const int s = swz128(row), c = 4 * half + 2 * fg + part;
  return *reinterpret_cast<const i32x4*>(tile + row * WBK + ((c ^ s) << 4));
}

// 32 bytes of row `row` at k = 64*half + 32*fg of a 128-byte-row tile.
__device__ __forceinline__ i32x8 frag128(const uint8_t* tile, int row, int fg, int half) {
  const int s = swz128(row), c = 4 * half + 2 * fg;
  return join(*reinterpret_cast<const i32x4*>(tile + row * WBK + ((c ^ s) << 4)),
              *reinterpret_cast<const i32x4*>(tile + row * WBK + (((c + 1) ^ s) << 4)));
}

// kStore: 0 = 2-byte stores, 1 = 8-byte stores (N % 4 == 0), 2 = through LDS with
// 16-byte row stores (N % 8 == 0, output 16-byte aligned).  kK128: K % 128 == 0 (copy_offset).
template <int kStore, bool kK128 = false>
__global__ __launch_bounds__(kThreads) void fp8_gemm_wide(
    const uint8_t* __restrict__ x, const uint8_t* __restrict__ w, int M, int N, int K,
    float inv_scale, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  int mt, nt;
  tile_of(blockIdx.x, tm, tn, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int rows_a = min(BM, M - m0), rows_b = min(BN, N - n0);
  const __amdgpu_buffer_rsrc_t xa = make_rsrc(x + (size_t)m0 * K, (size_t)rows_a * K);
  const __amdgpu_buffer_rsrc_t wb = make_rsrc(w + (size_t)n0 * K, (size_t)rows_b * K);

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  const int nk = (K + WBK - 1) / WBK;
  // Copies past the last step have offsets past K: the descriptor zero-fills the (free)
  // slot without touching memory, so the loop needs no branches (a branch around the
  // MFMAs would make the compiler copy the accumulators).
  auto a_tile = [&](int step) { return smem + (step % 3) * kWideOperandBytes; };
  auto b_tile = [&](int step) { return smem + (3 + (step & 1)) * kWideOperandBytes; };
  // The wave index as a scalar: each copy's LDS destination (M0) is then scalar arithmetic.
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  auto copy_a = [&](int step, int g0, int n) {
    dma_tile128<kK128>(xa, a_tile(step), rows_a, K, step * WBK, wave_s, lane, g0, n);
  };
  auto copy_b = [&](int step, int g0, int n) {
    dma_tile128<kK128>(wb, b_tile(step), rows_b, K, step * WBK, wave_s, lane, g0, n);
  };
  const int fr = lane % 32, fg = lane / 32;
  const int arow = wm * WM + fr, brow = wn * WN + fr;

  // Prologue: steps 0 and 1 (x then w each), then step 0's first-half fragments.
  copy_a(0, 0, kWideDmaPerWave);
  copy_b(0, 0, kWideDmaPerWave);
  copy_a(1, 0, kWideDmaPerWave);
  copy_b(1, 0, kWideDmaPerWave);
  wait_vmcnt<2 * kWideDmaPerWave>();
  __syncthreads();
  i32x8 a0[4], b0[4], a1[4], b1[4];  // first and second half of a step
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    b0[i] = frag128(b_tile(0), brow + 32 * i, fg, 0);
    a0[i] = frag128(a_tile(0), arow + 32 * i, fg, 0);
  }

  for (int kt = 0; kt < nk; ++kt) {
    // First half: MFMAs on (a0, b0) while the second half's fragments are read and step
    // kt+2's x copies go out, each MFMA with one 16-byte read and every other one a copy
    // (here after the odd MFMAs; in the second half after the even MFMAs of even rows and
    // the odd ones of odd rows: together 5-6 % faster than after the even ones throughout).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      i32x4 part[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[i][j] = mfma32_e4m3(b0[j], a0[i], acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);  // the MFMA issues before its copy
        if (j % 2 == 1) copy_a(kt + 2, 2 * i + j / 2, 1);
        part[j] = j < 2 ? frag128_part(b_tile(kt), brow + 32 * i, fg, 1, j)
                        : frag128_part(a_tile(kt), arow + 32 * i, fg, 1, j - 2);
        __builtin_amdgcn_sched_barrier(0);
      }
      b1[i] = join(part[0], part[1]);
      a1[i] = join(part[2], part[3]);
    }
    // Step kt+1 landed (only step kt+2's x copies, issued since, may be outstanding), and
    // every wave holds step kt in registers.
    wait_vmcnt<kWideDmaPerWave>();
    barrier_no_vm_drain();
    // Second half: MFMAs on (a1, b1) while step kt+1's first-half fragments are read and
    // step kt+2's w copies go out into the slot step kt just left.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      i32x4 part[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[i][j] = mfma32_e4m3(b1[j], a1[i], acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);  // the MFMA issues before its copy
        if (j % 2 == i % 2) copy_b(kt + 2, 2 * i + j / 2, 1);
        part[j] = j < 2 ? frag128_part(b_tile(kt + 1), brow + 32 * i, fg, 0, j)
                        : frag128_part(a_tile(kt + 1), arow + 32 * i, fg, 0, j - 2);
        __builtin_amdgcn_sched_barrier(0);
      }
      b0[i] = join(part[0], part[1]);
      a0[i] = join(part[2], part[3]);
    }
  }
  // The bias (L2-resident) is loaded only now: no LDS is free during the loop and a
  // register held through it would spill.
  const unsigned short bias_v = load_bias(bias, n0, rows_b, tid);
  // bias_s lies in w slot 1, where the zero-filling copies of step nk+1 land when nk is
  // even, and each wave's vmcnt covers only its own copies: every wave drains its copies
  // and passes a barrier before any wave writes the bias there.
  wait_vmcnt<0>();
  __syncthreads();
  uint16_t* bias_s = reinterpret_cast<uint16_t*>(smem + BM * kTileRowBytes);
  bias_s[tid] = bias_v;
  __syncthreads();
  // The epilogue's thread indices come from an opaque copy of tid, so the compiler cannot
  // compute them before the loop and carry them through it (where no register is free).
  int et = tid;
  asm volatile("" : "+v"(et));
  const int ew = et / kWave, el = et % kWave;
  const int ewm = ew / kWavesN, ewn = ew % kWavesN, efr = el % 32, efg = el / 32;
  if constexpr (kStore == 2)
    store_tile_lds(acc, out, bias_s, smem, N, m0, n0, ewm, ewn, efr, efg, rows_a, rows_b, inv_scale, et);
  else
    store_transposed_block<kStore == 1>(acc, out, bias_s, N, m0, n0, ewm, ewn, efr, efg, rows_a, inv_scale);
}

// ---------------------------------------------------------------------------------------
// Half-height wide kernel: 128x256 output tiles (128 x rows, 256 w rows) for grids in
// which 256x256 tiles would leave half the CUs or more idle (M = 2048, N = 4096 is 128
// such tiles on 256 CUs).  Same copies, fragment layout, 32x32x64 MFMAs and epilogues as
// fp8_gemm_wide; the 4 waves are arranged 2 (x) x 2 (w) with 64x128 wave tiles (2 x 4
// blocks).  A step now moves 16 KiB of x and 32 KiB of w for half the MFMAs, so both
// operands get a three-slot ring (3 x 16 + 3 x 32 = 144 KiB) and each wave's 12 copies of
// step kt+2 are spread evenly over the 16 MFMAs of step kt, all into the slots step kt-1
// left (every wave passed the barrier at step kt-1's mid-step, after its last read of
// them).  The 12 16-byte fragment reads of each half step (4 w blocks and 2 x blocks, two
// parts each) ride on its 8 MFMAs, one or two per MFMA.  Accumulation order is the same
// k-ascending sequence of 64-wide MFMA steps as the 256-row kernel, so the two give the
// same bits.
// ---------------------------------------------------------------------------------------
constexpr int kHalfRows = 128;                                      // x rows per tile
constexpr int kHalfMI = kHalfRows / 64;                             // 32-row x blocks per wave: 2
constexpr int kHalfXBytes = kHalfRows * WBK;                        // 16 KiB of x per step
constexpr int kHalfLdsBytes = 3 * (kHalfXBytes + kWideOperandBytes);  // 144 KiB
constexpr int kHalfXDma = kHalfRows / 8 / (kThreads / kWave);       // x copies per wave and step: 4
constexpr int kHalfCopies = kHalfXDma + kWideDmaPerWave;             // 12
constexpr int kHalfParts = 2 * (4 + kHalfMI);                        // 16-byte reads per half step: 12
constexpr int kHalfSlots = 4 * kHalfMI;                              // MFMAs per half step: 8
static_assert(kHalfRows * kTileRowBytes <= kHalfLdsBytes, "the output tile fits the rings");
// The bias sits past the rings, where no copy lands.
constexpr int kHalfLaunchLdsBytes = kHalfLdsBytes + kBiasBytes;  // 144.5 KiB
static_assert(kHalfCopies % 2 == 0, "each half step issues half the copies");

// Group `group` (8 rows) of a tile with 128-byte rows: one direct-to-LDS instruction.
template <bool kK128>
__device__ __forceinline__ void dma_group128(__amdgpu_buffer_rsrc_t r, uint8_t* lds_tile, int rows, int K,
                                             int k0, int group, int lane) {
  const int row = group * 8 + lane / 8;
  const int gk = k0 + 16 * ((lane % 8) ^ swz128(row));
  const unsigned off = copy_offset<kK128>(row, rows, gk, K);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)(lds_tile + group * kSlotsPerInst * 16), 16, off, 0, 0, 0);
}

template <int kStore, bool kK128 = false>
__global__ __launch_bounds__(kThreads) void fp8_gemm_half(
    const uint8_t* __restrict__ x, const uint8_t* __restrict__ w, int M, int N, int K,
    float inv_scale, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tm = (M + kHalfRows - 1) / kHalfRows, tn = (N + BN - 1) / BN;
  int mt, nt;
  tile_of(blockIdx.x, tm, tn, mt, nt);
  const int m0 = mt * kHalfRows, n0 = nt * BN;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int rows_a = min(kHalfRows, M - m0), rows_b = min(BN, N - n0);
  const __amdgpu_buffer_rsrc_t xa = make_rsrc(x + (size_t)m0 * K, (size_t)rows_a * K);
  const __amdgpu_buffer_rsrc_t wb = make_rsrc(w + (size_t)n0 * K, (size_t)rows_b * K);

  f32x16 acc[kHalfMI][4];
#pragma unroll
  for (int i = 0; i < kHalfMI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  const int nk = (K + WBK - 1) / WBK;
  // As in fp8_gemm_wide, copies past the last step zero-fill a free slot.
  auto a_tile = [&](int step) { return smem + (step % 3) * kHalfXBytes; };
  auto b_tile = [&](int step) { return smem + 3 * kHalfXBytes + (step % 3) * kWideOperandBytes; };
  // Copy c (0 .. 11) of this wave for `step`: x groups first, then w groups.  The wave
  // index is a scalar, so each copy's LDS destination (M0) is scalar arithmetic.
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  auto copy = [&](int step, int c) {
    if (c < kHalfXDma)
      dma_group128<kK128>(xa, a_tile(step), rows_a, K, step * WBK, wave_s * kHalfXDma + c, lane);
    else
      dma_group128<kK128>(wb, b_tile(step), rows_b, K, step * WBK, wave_s * kWideDmaPerWave + c - kHalfXDma, lane);
  };
  const int fr = lane % 32, fg = lane / 32;
  const int arow = wm * 32 * kHalfMI + fr, brow = wn * WN + fr;
  // 16-byte part p of `half` of step `step`: parts 0..7 are w blocks 0..3, 8..11 x blocks.
  auto part_of = [&](int step, int p, int half) {
    return p < 8 ? frag128_part(b_tile(step), brow + 32 * (p / 2), fg, half, p % 2)
                 : frag128_part(a_tile(step), arow + 32 * ((p - 8) / 2), fg, half, p % 2);
  };

  // Prologue: the bias (staged past the rings, so its load overlaps the first copies'),
  // steps 0 and 1, then step 0's first-half fragments.
  const unsigned short bias_v = load_bias(bias, n0, rows_b, tid);
#pragma unroll
  for (int c = 0; c < kHalfCopies; ++c) copy(0, c);
#pragma unroll
  for (int c = 0; c < kHalfCopies; ++c) copy(1, c);
  wait_vmcnt<kHalfCopies>();
  uint16_t* bias_s = reinterpret_cast<uint16_t*>(smem + kHalfLdsBytes);
  bias_s[tid] = bias_v;
  __syncthreads();
  i32x8 a0[kHalfMI], b0[4], a1[kHalfMI], b1[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) b0[j] = frag128(b_tile(0), brow + 32 * j, fg, 0);
#pragma unroll
  for (int i = 0; i < kHalfMI; ++i) a0[i] = frag128(a_tile(0), arow + 32 * i, fg, 0);

  // One half step: the MFMAs on (a, b), copies c0 .. c0+5 of step kt+2 and the parts of
  // `half` of step `rstep` into (na, nb).
  auto half_step = [&](const i32x8 (&a)[kHalfMI], const i32x8 (&b)[4], i32x8 (&na)[kHalfMI], i32x8 (&nb)[4],
                       int kt, int c0, int rstep, int half) {
    i32x4 part[kHalfParts];
#pragma unroll
    for (int s = 0; s < kHalfSlots; ++s) {
      const int i = s / 4, j = s % 4;
      acc[i][j] = mfma32_e4m3(b[j], a[i], acc[i][j]);
#pragma unroll
      for (int c = (kHalfCopies / 2) * s / kHalfSlots; c < (kHalfCopies / 2) * (s + 1) / kHalfSlots; ++c)
        copy(kt + 2, c0 + c);
#pragma unroll
      for (int p = kHalfParts * s / kHalfSlots; p < kHalfParts * (s + 1) / kHalfSlots; ++p)
        part[p] = part_of(rstep, p, half);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) nb[j] = join(part[2 * j], part[2 * j + 1]);
#pragma unroll
    for (int i = 0; i < kHalfMI; ++i) na[i] = join(part[8 + 2 * i], part[9 + 2 * i]);
  };

  for (int kt = 0; kt < nk; ++kt) {
    // First half: MFMAs on step kt's first 64 k, reading its second 64 k.
    half_step(a0, b0, a1, b1, kt, 0, kt, 1);
    // Step kt+1 landed (only step kt+2's first six copies may be outstanding), and every
    // wave holds step kt in registers.
    wait_vmcnt<kHalfCopies / 2>();
    barrier_no_vm_drain();
    // Second half: MFMAs on step kt's second 64 k, reading step kt+1's first 64 k.
    half_step(a1, b1, a0, b0, kt, kHalfCopies / 2, kt + 1, 0);
  }
  // The output tile is staged in the rings: every wave drains its own copies (the
  // zero-filling ones past K included) and passes a barrier before any wave writes there.
  wait_vmcnt<0>();
  __syncthreads();
  int et = tid;
  asm volatile("" : "+v"(et));
  const int ew = et / kWave, el = et % kWave;
  const int ewm = ew / kWavesN, ewn = ew % kWavesN, efr = el % 32, efg = el / 32;
  if constexpr (kStore == 2)
    store_tile_lds<kHalfMI>(acc, out, bias_s, smem, N, m0, n0, ewm, ewn, efr, efg, rows_a, rows_b, inv_scale, et);
  else
    store_transposed_block<kStore == 1, kHalfMI>(acc, out, bias_s, N, m0, n0, ewm, ewn, efr, efg, rows_a, inv_scale);
}

// ---------------------------------------------------------------------------------------
// Skinny kernel (M <= 64)
// ---------------------------------------------------------------------------------------
constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyThreads = kSkinnyWaves * kWave;
constexpr int kSkinnyMaxM = 64;

// Column block of workgroup b among nb: a bf16 output line (64 columns) is four 16-column
// blocks, and workgroups are dispatched round-robin over the 8 XCDs, so XCD x's workgroups
// b = x + 8 j take whole lines, 4 (x + 8 (j / 4)) + j % 4, and a line's four partial writes
// merge in one L2 (a bijection on the first 32 floor(nb / 32) blocks; the rest keep their
// index).  Dispatch order only affects speed, never which outputs are written.
__device__ __forceinline__ int skinny_block(int b, int nb) {
  if (b >= nb / 32 * 32) return b;
  const int x = b % 8, j = b / 8;
  return 4 * (x + 8 * (j / 4)) + j % 4;
}

template <int kVec>
__global__ __launch_bounds__(kSkinnyThreads) void fp8_gemm_skinny(
    const uint8_t* __restrict__ x, const uint8_t* __restrict__ w, int M, int N, int K,
    float inv_scale, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out) {
  __shared__ float part[kSkinnyWaves][kSkinnyMaxM][16];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int n0 = skinny_block(blockIdx.x, gridDim.x) * 16;
  const int fr = lane % 16, fg = lane / 16;
  const int rblocks = (M + 15) / 16;
  const int steps = (K + 127) / 128;
  const int per_wave = (steps + kSkinnyWaves - 1) / kSkinnyWaves;
  const int s0 = wave * per_wave, s1 = min(steps, s0 + per_wave);

  f32x4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int rows_w = min(16, N - n0);
  const __amdgpu_buffer_rsrc_t wb = make_rsrc(w + (size_t)n0 * K, (size_t)rows_w * K);
  const __amdgpu_buffer_rsrc_t xa = make_rsrc(x, (size_t)M * K);
  const unsigned woff = fr < rows_w ? (unsigned)(fr * K) : kOutOfRange;
  for (int s = s0; s < s1; ++s) {
    const int k = s * 128 + 32 * fg;
    const unsigned wo = woff == kOutOfRange ? kOutOfRange : woff + k;
    const i32x8 bf = join(load16<kVec>(wb, wo, k, K), load16<kVec>(wb, wo + 16, k + 16, K));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i < rblocks) {
        const int gm = i * 16 + fr;
        const unsigned xo = gm < M ? (unsigned)(gm * K + k) : kOutOfRange;
        const i32x8 af = join(load16<kVec>(xa, xo, k, K), load16<kVec>(xa, xo + 16, k + 16, K));
        acc[i] = mfma_e4m3(af, bf, acc[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (i < rblocks)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[wave][i * 16 + 4 * fg + r][fr] = acc[i][r];
  __syncthreads();
  for (int e = threadIdx.x; e < M * 16; e += kSkinnyThreads) {
    const int m = e / 16, c = e % 16;
    const int n = n0 + c;
    if (n >= N) continue;
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < kSkinnyWaves; ++v) s += part[v][m][c];
    out[(size_t)m * N + n] = f32_to_bf16_rne(s * inv_scale + bf16_to_f32(bias[n]));
  }
}

// ---------------------------------------------------------------------------------------
// Skinny kernel, 16-byte path (M <= 64, K % 16 == 0, 16-byte aligned x and w).
//
// Same work split as fp8_gemm_skinny: a workgroup owns 16 output columns and all M rows,
// its 8 waves split K, and the partial tiles are reduced through LDS in wave order.  The
// MFMA layout has each load instruction touch 16 rows K bytes apart (4 lanes per row), and
// on MI355X that weight stream ran at 5.2 us for 16 MiB against 4.0 us for whole 1 KiB
// runs, since rows a power of two apart fall on the same L2 channel.  So each wave loads
// its kSl-byte K slice of the 16 W rows and of the M x rows as flat runs (kSl / 16 lanes
// per row), writes them into its own LDS region (row r's 16-byte chunk c at chunk
// c ^ (r % kSwz), which spreads both the row writes and the fragment reads over the
// banks), and reads the MFMA fragments back.  Wave w takes k0 = kSl * (w + 8j): for
// K = 4096 and kSl = 512 that is the same K range, in the same step order, as
// fp8_gemm_skinny's wave w.
// ---------------------------------------------------------------------------------------
constexpr int skinny_slice(int rb) { return rb == 1 ? 512 : rb <= 3 ? 256 : 128; }
constexpr int skinny_lds_bytes(int rb) {
  return kSkinnyWaves * (16 + 16 * rb) * skinny_slice(rb) + kSkinnyWaves * 16 * rb * 16 * 4;
}

template <int kRB>  // row blocks of 16: M <= 16 * kRB
__global__ __launch_bounds__(kSkinnyThreads) void fp8_gemm_skinny_flat(
    const uint8_t* __restrict__ x, const uint8_t* __restrict__ w, int M, int N, int K,
    float inv_scale, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out) {
  constexpr int kSl = skinny_slice(kRB);
  constexpr int kChunks = kSl / 16;                  // 16-byte chunks per slice row
  constexpr int kSwz = kChunks < 16 ? kChunks : 16;  // chunk swizzle period
  constexpr int kRowsPerLoad = kWave / kChunks;      // rows one load instruction covers
  constexpr int kRows = 16 + 16 * kRB;               // W rows, then x rows
  constexpr int kLoads = kRows / kRowsPerLoad;
  constexpr int kSteps = kSl / 128;                  // MFMA k-steps per slice
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int n0 = skinny_block(blockIdx.x, gridDim.x) * 16;
  const int fr = lane % 16, fg = lane / 16;
  uint8_t* mine = smem + wave * kRows * kSl;
  float* part = reinterpret_cast<float*>(smem + kSkinnyWaves * kRows * kSl);  // [wave][16 kRB][16]
  const int rows_w = min(16, N - n0);
  const __amdgpu_buffer_rsrc_t wb = make_rsrc(w + (size_t)n0 * K, (size_t)rows_w * K);
  const __amdgpu_buffer_rsrc_t xa = make_rsrc(x, (size_t)M * K);
  const int lr = lane / kChunks, p = lane % kChunks;  // row within a load, chunk
  // Every output this thread finishes is in column n0 + tid % 16 (the epilogue's stride is
  // a multiple of 16), so its bias is loaded now and its latency overlaps the K loop's.
  const int bc = (int)threadIdx.x % 16;
  const __amdgpu_buffer_rsrc_t rbias = make_rsrc(bias + n0, (size_t)rows_w * 2);
  const float bias_v = bf16_to_f32(
      __builtin_amdgcn_raw_buffer_load_b16(rbias, bc < rows_w ? (unsigned)bc * 2u : kOutOfRange, 0, 0));
  f32x4 acc[kRB];
#pragma unroll
  for (int i = 0; i < kRB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = wave * kSl; k0 < K; k0 += kSkinnyWaves * kSl) {
    const bool kin = k0 + 16 * p < K;  // K % 16 == 0: a chunk is wholly inside or past K
    i32x4 v[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int r = i * kRowsPerLoad + lr;
      if (r < 16) {
        // W is streamed once (each row by one workgroup): non-temporal loads.  Same bits;
        // M = 16: 6.15 -> 5.93-5.95 us per call (A/B on one box, both orders).  x, which
        // every workgroup reads, keeps the default policy.
        const unsigned off = (kin && r < rows_w) ? (unsigned)(r * K + k0 + 16 * p) : kOutOfRange;
        v[i] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(wb, off, 0, kCachePolicyNT));
      } else {
        const unsigned off = (kin && r - 16 < M) ? (unsigned)((r - 16) * K + k0 + 16 * p) : kOutOfRange;
        v[i] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(xa, off, 0, 0));
      }
    }
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int r = i * kRowsPerLoad + lr;
      *reinterpret_cast<i32x4*>(mine + r * kSl + ((p ^ (r % kSwz)) << 4)) = v[i];
    }
    auto frag = [&](int row, int u) {
      const int c = 8 * u + 2 * fg, s = row % kSwz;
      return join(*reinterpret_cast<const i32x4*>(mine + row * kSl + ((c ^ s) << 4)),
                  *reinterpret_cast<const i32x4*>(mine + row * kSl + (((c + 1) ^ s) << 4)));
    };
#pragma unroll
    for (int u = 0; u < kSteps; ++u) {
      const i32x8 bf = frag(fr, u);
#pragma unroll
      for (int i = 0; i < kRB; ++i) acc[i] = mfma_e4m3(frag(16 + 16 * i + fr, u), bf, acc[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < kRB; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) part[(wave * 16 * kRB + i * 16 + 4 * fg + r) * 16 + fr] = acc[i][r];
  __syncthreads();
  for (int e = threadIdx.x; e < M * 16; e += kSkinnyThreads) {
    const int m = e / 16, c = e % 16, n = n0 + c;
    if (n >= N) continue;
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < kSkinnyWaves; ++q) s += part[(q * 16 * kRB + m) * 16 + c];
    out[(size_t)m * N + n] = f32_to_bf16_rne(s * inv_scale + bias_v);
  }
}

inline int vec_width(const uint8_t* x, const uint8_t* w, int K) {
  const uintptr_t bits = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w);
  if (K % 16 == 0 && (bits & 15) == 0) return 16;
  if (K % 8 == 0 && (bits & 7) == 0) return 8;
  return 1;
}

}  // namespace fp8
}  // namespace taskops
