// efficient_kan kernels for gfx950 (instantiated by efficient_kan.hip).
//
// Op: tasks/efficient_kan/reference.py:33-51 (fp64 oracle :54-57):
//   out[b,o] = sum_i silu(x[b,i]) Wb[o,i] + sum_i sum_c B_c(x[b,i]) Ws[o,i,c] sc[o,i]
// with B_c the order-p B-spline bases on feature i's knot row (Cox-de Boor).
//
// One contraction over K = I * (1 + C') (C' = C rounded up to 8 or 16) on the fp16 MFMA
// v_mfma_f32_16x16x32_f16 with a three-term split for fp32-level accuracy: every operand v
// is carried as hi = fp16(v) and lo = fp16(v - hi), and each product as hi*hi + lo*hi +
// hi*lo (the dropped lo*lo term is ~2^-22 relative), accumulated in fp32.
//
// K order: features in groups of 32; each group is one "silu" chunk (32 features, k =
// feature) followed by C' "spline" chunks; spline chunk t holds the C' bases of the 32/C'
// features i*C' + t (k = i*C' + basis).  In MFMA layout lane l supplies k = 8*(l/16) .. +7
// of batch row l % 16, so over one group a lane needs x at one contiguous run of C'
// features, and in a spline chunk it owns one (row, feature) and 8 of its bases: it finds
// x's knot interval, evaluates the four bases nonzero there from per-interval cubic
// coefficients and shifts them into its 8 slots.
//
// Per call, two launches: kan_pack finds each output column's power-of-two scale (so
// neither fp16 half under- or overflows), writes the weights ([Wb | Ws*sc], the A operand)
// in that K order as scaled fp16 hi/lo, [chunk][column][32] so each chunk's tile is
// contiguous, and tabulates every feature's knot row and per-interval basis cubics;
// kan_fused is the warp-specialized GEMM (producer waves copy weight tiles and expand
// activations into LDS, consumer waves run the MFMAs) and undoes the column scale in its
// epilogue.
#pragma once

#include <utility>

#include "common.hpp"

namespace taskops {
namespace kan {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kGroup = 32;        // features per group
constexpr int kChunk = 32;        // k per MFMA chunk
constexpr int kMaxKnots = 16;     // fast path: grid_size + 2*order + 1 <= 16
constexpr int kOrder = 3;         // the fast path's spline order
constexpr int kRawBufferFlags = 0x00020000;
constexpr unsigned kOutOfRange = 0x80000000u;

// kan_fused tiling: a 128 x 256 output tile per workgroup of 8 waves.  Waves 0-3 are
// consumers: wave w owns all 128 batch rows (8 row blocks of 16) x output columns
// 64w .. 64w+63 (4 column blocks), 128 fp32 accumulators, and only reads LDS and issues
// MFMAs.  Waves 4-7 are producers: producer p copies a quarter of each weight tile into
// LDS and expands the activations of batch rows 32p .. 32p+31 (2 row blocks).  One
// producer and one consumer share each SIMD.
constexpr int kThreads = 512;
constexpr int kConsumerWaves = 4;
constexpr int BM = 128;
constexpr int BN = 256;
constexpr int kRB = BM / 16;                        // row blocks per tile (consumer)
constexpr int kCB = BN / 16 / kConsumerWaves;       // column blocks per consumer wave
constexpr int kWHalfBytes = BN * kChunk * 2;        // hi or lo weights of one chunk: 16 KiB
constexpr int kWStageBytes = 2 * kWHalfBytes;       // one chunk's weight tile: 32 KiB
constexpr int kWStages = 3;                         // weight ring: copies run two chunks ahead
constexpr int kActBytes = kRB * 2 * 64 * 16;        // hi + lo activation fragments: 16 KiB
constexpr int kActStages = 2;
constexpr int kActAt = kWStages * kWStageBytes;
constexpr int kTblAt = kActAt + kActStages * kActBytes;
constexpr int kTblBytes = 32 * 1024;                // one group's table (L <= 16)
constexpr int kLdsBytes = kTblAt + kTblBytes;       // 160 KiB
static_assert(kLdsBytes <= 160 * 1024, "fits one CU's LDS");

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, size_t bytes) {
  const int n = bytes > 0x7fffffffu ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, kRawBufferFlags);
}

// Padded basis count C' for C bases (8, 16 or 32; 0 when C > 32).
inline int padded_bases(int C) { return C <= 8 ? 8 : (C <= 16 ? 16 : (C <= 32 ? 32 : 0)); }

// ---------------------------------------------------------------------------------------
// Basis tables: for every feature, its knot row (16 floats, +inf past L) followed by, for
// each knot interval j in [0, L-1), the cubic coefficients of the four bases j-3..j that
// are nonzero on [t_j, t_{j+1}), as polynomials in u = x - t_j (16 floats: basis c's
// c0..c3 in 16-byte chunk tbl_chunk(j, c % 4)).  A basis outside [0, C) has zero
// coefficients.  The polynomials come from the Cox-de Boor recursion carried out on
// polynomials in fp64 with the reference's index ranges (tasks/efficient_kan/
// reference.py:33-39: N_{k,p} exists for 0 <= k <= L-2-p); a zero-width knot span
// contributes nothing.  Layout: [group][tbl_group_bytes], feature fl of a group at
// fl * 64 * L bytes, so one group is one contiguous copy.
// ---------------------------------------------------------------------------------------
__host__ __device__ inline int tbl_group_bytes(int L) { return 4096 * ((L + 1) / 2); }

// Position of basis r's 16-byte coefficient chunk within interval j's 64 bytes: XOR-ed
// with (j >> 2) & 3, so lanes of one feature reading intervals j and j + 4 (the same banks
// at a 64-byte stride) hit different banks.
__host__ __device__ inline int tbl_chunk(int j, int r) { return r ^ ((j >> 2) & 3); }

// Entry j of a feature's table (dst: the feature's 16 * L floats): j = -1 writes the knot
// row, j in [0, L-1) interval j's cubics.
__host__ __device__ void kan_table_entry(const float* __restrict__ knots_row, int L, int j, float* __restrict__ dst) {
  if (j < 0) {
    for (int k = 0; k < kMaxKnots; ++k) dst[k] = k < L ? knots_row[k] : __builtin_inff();
    return;
  }
  double t[kMaxKnots];
  for (int k = 0; k < kMaxKnots; ++k) t[k] = k < L ? (double)knots_row[k] : 0.0;
  double P[kOrder + 1][4];  // P[r]: N_{j-3+r, p} as a cubic in u
  for (int r = 0; r <= kOrder; ++r)
    for (int c = 0; c < 4; ++c) P[r][c] = 0.0;
  if (t[j + 1] > t[j]) P[kOrder][0] = 1.0;  // N_{j,0} on [t_j, t_{j+1})
  for (int p = 1; p <= kOrder; ++p) {
    double Q[kOrder + 1][4];
    for (int r = 0; r <= kOrder; ++r) {
      for (int c = 0; c < 4; ++c) Q[r][c] = 0.0;
      const int k = j - kOrder + r;
      if (r < kOrder - p || k < 0 || k > L - 2 - p) continue;
      const double d1 = t[k + p] - t[k], d2 = t[k + p + 1] - t[k + 1];
      if (d1 != 0.0) {  // (u + (t_j - t_k)) / d1 * N_{k,p-1}
        const double a = (t[j] - t[k]) / d1, b = 1.0 / d1;
        for (int c = 3; c >= 0; --c) Q[r][c] += a * P[r][c] + (c > 0 ? b * P[r][c - 1] : 0.0);
      }
      if (d2 != 0.0 && r < kOrder) {  // ((t_{k+p+1} - t_j) - u) / d2 * N_{k+1,p-1}
        const double a = (t[k + p + 1] - t[j]) / d2, b = -1.0 / d2;
        for (int c = 3; c >= 0; --c) Q[r][c] += a * P[r + 1][c] + (c > 0 ? b * P[r + 1][c - 1] : 0.0);
      }
    }
    for (int r = 0; r <= kOrder; ++r)
      for (int c = 0; c < 4; ++c) P[r][c] = Q[r][c];
  }
  for (int r = 0; r <= kOrder; ++r)  // basis j - 3 + r; (j - 3 + r) % 4 == (j + 1 + r) % 4
    for (int c = 0; c < 4; ++c) dst[kMaxKnots + j * 16 + 4 * tbl_chunk(j, (j + 1 + r) & 3) + c] = (float)P[r][c];
}

// Whether a knot row is uniform enough for the GEMM's direct interval lookup: h > 0 and
// every knot within 1e-3 h of t_0 + k h (the grids efficient-kan builds, arange * h + a
// in fp32, are uniform to a few ulps).
__host__ __device__ inline bool kan_knots_uniform(const float* __restrict__ t, int L) {
  if (L < 2) return false;
  const double h = ((double)t[L - 1] - (double)t[0]) / (L - 1);
  if (!(h > 0.0) || !(h < 1e300)) return false;
  for (int k = 0; k < L; ++k)
    if (!(__builtin_fabs((double)t[k] - ((double)t[0] + k * h)) <= 1e-3 * h)) return false;
  return true;
}

// ---------------------------------------------------------------------------------------
// Weight preparation, one launch (kan_pack): each output column's scale, the GEMM's A
// operand, and the basis tables.
// bhi/blo: [nchunks][Opad][32] fp16; chunk q = g*(1+Cp) + sub; sub 0 holds Wb[o, 32g + s],
// sub >= 1 holds (Ws*sc)[o, f, c] with f = 32g + (s/Cp)*Cp + (sub-1), c = s % Cp (zero
// past I, O or C), all times 2^e.  So over a group's spline chunks the lanes that supply
// slots s..s+7 of a chunk walk the features (s/Cp)*Cp .. +Cp-1: the same 8 (Cp = 8) or 16
// features whose silu values they supply, and the GEMM loads each lane's x values as one
// contiguous run.  colscale[o] = 2^-e with e chosen so max|column| * 2^e is in
// [2^14, 2^15), so neither fp16 half under- or overflows.
// ---------------------------------------------------------------------------------------
// Basis tables, one thread per table entry (L per feature: the knot row and the L - 1
// intervals), kThreadsPerBlock entries per workgroup; uflags[block] = 1 when every knot
// row the block wrote is uniform (kan_knots_uniform), else 0.
template <int kThreadsPerBlock>
__device__ __forceinline__ void kan_tables_block(int block, const float* __restrict__ grid, int I, int L,
                                                 int ngroups, float* __restrict__ tables,
                                                 int* __restrict__ uflags) {
  const int idx = block * kThreadsPerBlock + (int)threadIdx.x;
  const int f = idx / L, j = idx % L - 1;
  bool uniform = true;
  if (f < ngroups * kGroup) {
    float* dst = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(tables) +
                                          (size_t)(f / kGroup) * tbl_group_bytes(L) + (f % kGroup) * 64 * L);
    if (f < I) {
      kan_table_entry(grid + (size_t)f * L, L, j, dst);
      if (j < 0) uniform = kan_knots_uniform(grid + (size_t)f * L, L);
    } else if (j < 0) {  // missing feature: knots 0, 1, 2, ... and zero coefficients
      for (int k = 0; k < kMaxKnots; ++k) dst[k] = (float)k;
    } else {
      for (int k = 0; k < 16; ++k) dst[kMaxKnots + 16 * j + k] = 0.0f;
    }
  }
  uniform = __syncthreads_and(uniform);
  if (threadIdx.x == 0) uflags[block] = uniform ? 1 : 0;
}

// kan_pack: the first tblocks workgroups build the basis tables (kan_tables_block); they
// need nothing from the packing, so they run beside it.  Workgroup tblocks + t owns output
// columns kPackCols*t .. +kPackCols-1 with kColWaves waves each; wave q of a column takes
// the runs of 64 features q*64 + 64*kColWaves*j (lane = feature within the run), so a
// wave's loads cover 64 consecutive features of the column's contiguous rows.  Pass 1
// reduces the column's max |w| over Wb, sc and Ws to colscale[o] (waves combine through
// LDS); pass 2 reads the column again (now from the L2 or the Infinity Cache) and writes its
// hi/lo weights: lane (column o, feature f) writes all of f's bases, one run of Cp slots
// (fl / Cp) * Cp .. in spline chunk 1 + fl % Cp of group f / 32 (fl = f % 32), and lanes
// with fl < 4 also write silu slots 8 fl .. +7.  Workgroup tblocks also zeroes kan_fused's
// split-K arrival counters (their place in the workspace moves with the shape, so every
// call starts them from zero).
constexpr int kPackCols = 2;
constexpr int kColWaves = 4;
constexpr int kPackThreads = kPackCols * kColWaves * kWave;
template <int kCp>
__global__ __launch_bounds__(kPackThreads) void kan_pack(
    const float* __restrict__ wb, const float* __restrict__ ws, const float* __restrict__ sc, int I,
    int O, int C, int Opad, float* __restrict__ colscale, _Float16* __restrict__ bhi,
    _Float16* __restrict__ blo, const float* __restrict__ grid, int L, int ngroups, int tblocks,
    float* __restrict__ tables, int* __restrict__ uflags, unsigned* __restrict__ counters,
    int ncounters) {
  static_assert(kCp % 8 == 0, "whole 8-slot runs");
  __shared__ float colmax[kPackCols][kColWaves];
  if ((int)blockIdx.x < tblocks) {
    kan_tables_block<kPackThreads>(blockIdx.x, grid, I, L, ngroups, tables, uflags);
    return;
  }
  constexpr int kSub = 1 + kCp;
  constexpr int kStride = kColWaves * kWave;  // features between a wave's runs
  const int t = (int)blockIdx.x - tblocks;
  if (t == 0)
    for (int i = threadIdx.x; i < ncounters; i += kPackThreads) counters[i] = 0u;
  const int lane = (int)threadIdx.x % kWave, wave = (int)threadIdx.x / kWave;
  const int oc = wave / kColWaves, q = wave % kColWaves;
  const int o = t * kPackCols + oc;
  const int first = q * kWave + lane;
  const bool col = o < O;
  const bool vec = C % 4 == 0 && (reinterpret_cast<uintptr_t>(ws) & 15) == 0;
  const float* wsc = ws + (size_t)o * I * C;
  // Ws[o, f, c] for c < kCp (zero past C), times s.
  auto spline_row = [&](int f, float s, float (&v)[kCp]) {
    const float* row = wsc + (size_t)f * C;
    if (vec) {
#pragma unroll
      for (int c4 = 0; c4 < kCp / 4; ++c4) {
        f32x4 w4 = {0.f, 0.f, 0.f, 0.f};
        if (4 * c4 < C) w4 = *reinterpret_cast<const f32x4*>(row + 4 * c4);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * c4 + e] = w4[e] * s;
      }
    } else {
#pragma unroll
      for (int c = 0; c < kCp; ++c) v[c] = c < C ? row[c] * s : 0.0f;
    }
  };

  // Pass 1: max over the column.  max_c |ws * s| = |s| * max_c |ws| exactly (rounding is
  // monotonic); a wave's runs go four at a time so each lane keeps its loads in flight.  The
  // last four runs stay in registers for pass 2.
  float mx = 0.0f;
  float wbv[4], scv[4], rows[4][kCp];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    wbv[u] = 0.0f;
    scv[u] = 0.0f;
#pragma unroll
    for (int c = 0; c < kCp; ++c) rows[u][c] = 0.0f;
  }
  if (col) {
    for (int f0 = first; f0 < I; f0 += 4 * kStride) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int f = f0 + u * kStride;
        wbv[u] = 0.0f;
        scv[u] = 0.0f;
#pragma unroll
        for (int c = 0; c < kCp; ++c) rows[u][c] = 0.0f;
        if (f < I) {
          wbv[u] = wb[(size_t)o * I + f];
          scv[u] = sc[(size_t)o * I + f];
          spline_row(f, 1.0f, rows[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float m = 0.0f;
#pragma unroll
        for (int c = 0; c < kCp; ++c) m = fmaxf(m, fabsf(rows[u][c]));
        mx = fmaxf(mx, fmaxf(fabsf(wbv[u]), fabsf(scv[u]) * m));
      }
    }
  }
  for (int off = kWave / 2; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
  if (lane == 0) colmax[oc][q] = mx;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kColWaves; ++w) mx = fmaxf(mx, colmax[oc][w]);
  int e = 0;
  if (mx > 0.0f && mx < __builtin_inff()) e = 14 - ilogbf(mx);
  e = e > 100 ? 100 : (e < -100 ? -100 : e);
  if (q == 0 && lane == 0) colscale[o] = ldexpf(1.0f, -e);
  const float scale = ldexpf(1.0f, e);  // 2^e, exact

  // Pass 2: the scaled hi/lo weights of every group (zero past I and O).
  auto put = [&](int g, int sub, int slot, const float* v) {
    f16x8 h8, l8;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float w = v[k] * scale;
      const _Float16 h = (_Float16)w;
      h8[k] = h;
      l8[k] = (_Float16)(w - (float)h);
    }
    const size_t dst = ((size_t)(g * kSub + sub) * Opad + o) * kChunk + slot;
    *reinterpret_cast<f16x8*>(bhi + dst) = h8;
    *reinterpret_cast<f16x8*>(blo + dst) = l8;
  };
  if (ngroups * kGroup <= 4 * kStride) {
    // One batch of runs covers every feature (I <= 1024): pass 1's registers hold the
    // column's data.  Lane f % 32 < 4 of a group takes the silu weights of features
    // 8 (f % 32) .. +7 from the lanes that loaded them (a group sits within one run).
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int f = first + u * kStride, g = f / kGroup, fl = f % kGroup;
      float v[kCp], silu[8];
#pragma unroll
      for (int c = 0; c < kCp; ++c) v[c] = rows[u][c] * scv[u];
#pragma unroll
      for (int k = 0; k < 8; ++k) silu[k] = __shfl(wbv[u], (lane & 32) + ((8 * (lane & 3) + k) & 31), kWave);
      if (f < ngroups * kGroup) {
#pragma unroll
        for (int h = 0; h < kCp / 8; ++h) put(g, 1 + fl % kCp, (fl / kCp) * kCp + 8 * h, v + 8 * h);
        if (fl < 4) put(g, 0, 8 * fl, silu);
      }
    }
    return;
  }
  for (int f0 = first; f0 < ngroups * kGroup; f0 += 2 * kStride) {
    float rows2[2][kCp], silu[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int f = f0 + u * kStride, g = f / kGroup, fl = f % kGroup;
#pragma unroll
      for (int c = 0; c < kCp; ++c) rows2[u][c] = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) silu[u][k] = 0.0f;
      if (col && f < I) spline_row(f, sc[(size_t)o * I + f], rows2[u]);
      if (fl < 4) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int f2 = g * kGroup + 8 * fl + k;
          if (col && f2 < I) silu[u][k] = wb[(size_t)o * I + f2];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int f = f0 + u * kStride, g = f / kGroup, fl = f % kGroup;
      if (f < ngroups * kGroup) {
#pragma unroll
        for (int h = 0; h < kCp / 8; ++h) put(g, 1 + fl % kCp, (fl / kCp) * kCp + 8 * h, rows2[u] + 8 * h);
        if (fl < 4) put(g, 0, 8 * fl, silu[u]);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Weight tiles: 64-byte rows (32 fp16 of k); chunk c of row r sits at chunk c ^ ((r >> 1)
// & 3), which spreads the 16 rows x 4 chunks of one fragment read over all banks
// (measured on MI355X: 141 B/clk/CU against 127 unswizzled or with (r >> 2) & 3).
__device__ __forceinline__ int swz_w(int row) { return (row >> 1) & 3; }
__device__ __forceinline__ int swizzle64(int row, int chunk) {
  return row * 64 + ((chunk ^ swz_w(row)) << 4);
}

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// hi = fp16(v), lo = fp16(v - hi), both round-to-nearest-even.  hi is converted two values
// per v_cvt_pk_f16_f32; v - hi is exact in fp32, so lo is the single rounding of it, which
// one v_fma_mix (fp16 hi operand, fp32 v, fp16 result) computes.  The empty asm pins v as
// one fp32 value: otherwise the compiler may fuse the producer's last multiply with the
// rounding of hi (one rounding of the exact product) while lo is still taken from the
// fp32-rounded v, and hi + lo then misses v by an fp16 ulp in rare cases.
__device__ __forceinline__ void split8(const float* v, f16x8& hi, f16x8& lo) {
#pragma unroll
  for (int s = 0; s < 8; s += 2) {
    float v0 = v[s], v1 = v[s + 1];
    asm volatile("" : "+v"(v0), "+v"(v1));
    const f16x2 h = __builtin_convertvector(f32x2{v0, v1}, f16x2);
    hi[s] = h.x;
    hi[s + 1] = h.y;
    lo[s] = (_Float16)__builtin_fmaf((float)h.x, -1.0f, v0);
    lo[s + 1] = (_Float16)__builtin_fmaf((float)h.y, -1.0f, v1);
  }
}

// Output tile of workgroup b: the tm x tn tiles in column-major order, so the workgroups
// of one XCD (b % 8, dispatched round-robin) share a column panel of the weights.
__device__ __forceinline__ void tile_of(int b, int tm, int tn, int& mt, int& nt) {
  const int T = tm * tn;
  const int v = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
  nt = v / tm;
  mt = v % tm;
}

// Interval lookup.  j is the knot interval (clamped to [0, L-2]) whose cubics are
// evaluated and `inside` says whether x lies in [t_0, t_{L-1}) at all (outside, every
// basis is zero).  The coefficient chunk m holds the basis with index = m (mod 4).
struct TabFetch {
  f32x4 c[4];
  float tj;
  int j;
  bool inside;
};

__device__ __forceinline__ void tab_fetch(TabFetch& r, const float* fe) {
  r.tj = fe[r.j];
  const f32x4* cf = reinterpret_cast<const f32x4*>(fe + kMaxKnots + 16 * r.j);
#pragma unroll
  for (int m = 0; m < 4; ++m) r.c[m] = cf[tbl_chunk(r.j, m)];
}

__device__ __forceinline__ void tab_knots(const float* fe, f32x4 (&kn)[4]) {
  const f32x4* k4 = reinterpret_cast<const f32x4*>(fe);
#pragma unroll
  for (int q = 0; q < 4; ++q) kn[q] = k4[q];
}

// Any knot row: j + 1 = the number of knots <= x (reference.py:36-37, x in [t_j, t_{j+1})).
__device__ __forceinline__ TabFetch tab_locate_count(float x, const f32x4 (&kn)[4], const float* fe, int L) {
  int cnt = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) cnt += (x >= kn[q].x) + (x >= kn[q].y) + (x >= kn[q].z) + (x >= kn[q].w);
  TabFetch r;
  r.j = min(max(cnt - 1, 0), L - 2);
  r.inside = cnt >= 1 && cnt <= L - 1;
  tab_fetch(r, fe);
  return r;
}

// Uniform knot rows (every knot within 1e-3 h of t_0 + k h): j = floor((x - t_0) / h),
// with 1/h from the first two knots.  It can differ from the count only for x within
// ~1e-3 h of a knot, where the cubic pieces on either side agree to (1e-3)^3 / 6 of a
// basis value (cubic B-splines are C2 at simple knots), so the two lookups give the same
// bases to well under the op's tolerance.
__device__ __forceinline__ TabFetch tab_locate_uniform(float x, float t0, float inv_h, const float* fe, int L) {
  const int j = (int)__builtin_floorf((x - t0) * inv_h);
  TabFetch r;
  r.j = min(max(j, 0), L - 2);
  r.inside = j == r.j;
  tab_fetch(r, fe);
  return r;
}

// Evaluates the four cubics at u = x - t_j, splits them into fp16 hi/lo and routes them to
// the lane's 8 slots (bases b0 .. b0+7).  Basis c sits in slot c - b0; the value of
// coefficient chunk m belongs to the one basis of the window [j-3, j] with index = m
// (mod 4), so it goes to slot m or m + 4 (b0 is a multiple of 8), or to neither when that
// basis belongs to the other lane (Cp = 16).  With Cp = 8 (b0 = 0) bases outside [0, 8)
// have zero coefficients, so only the routing is needed: chunk m goes to slot m + 4
// exactly when m < j - 3.
template <int kCp>
__device__ __forceinline__ void tab_finish(float x, const TabFetch& t, int b0, f16x8& hi, f16x8& lo) {
  const float u = x - t.tj;
  float N[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const f32x4 c = t.c[m];
    N[m] = t.inside ? fmaf(fmaf(fmaf(c.w, u, c.z), u, c.y), u, c.x) : 0.0f;
  }
  asm volatile("" : "+v"(N[0]), "+v"(N[1]), "+v"(N[2]), "+v"(N[3]));
  const f16x2 h01 = __builtin_convertvector(f32x2{N[0], N[1]}, f16x2);
  const f16x2 h23 = __builtin_convertvector(f32x2{N[2], N[3]}, f16x2);
  // lo = fp16(N - hi), the difference exact in fp32: one v_fma_mix per value.
  f16x2 l01, l23;
  l01.x = (_Float16)__builtin_fmaf((float)h01.x, -1.0f, N[0]);
  l01.y = (_Float16)__builtin_fmaf((float)h01.y, -1.0f, N[1]);
  l23.x = (_Float16)__builtin_fmaf((float)h23.x, -1.0f, N[2]);
  l23.y = (_Float16)__builtin_fmaf((float)h23.y, -1.0f, N[3]);
  const unsigned H0 = __builtin_bit_cast(unsigned, h01), H1 = __builtin_bit_cast(unsigned, h23);
  const unsigned L0 = __builtin_bit_cast(unsigned, l01), L1 = __builtin_bit_cast(unsigned, l23);
  unsigned m0, m1, m2, m3;  // slot masks: slots 2d, 2d+1 take fp16 halves of dword d % 2
  if constexpr (kCp == 8) {
    const int k = min(max(t.j - kOrder, 0), 4);  // chunks m < k go to slots m + 4
    const unsigned long long M = k < 4 ? (~0ull << (16 * k)) : 0ull;
    m0 = (unsigned)M;
    m1 = (unsigned)(M >> 32);
    m2 = ~m0;
    m3 = ~m1;
  } else {
    // Slot s is live iff s in [p, p+3], p = j - 3 - b0 in [-11, 11]: bit s of `act`.
    const int p = t.j - kOrder - b0;
    const unsigned act = (0xFu << (p + 11)) >> 11;
    auto pair = [&](int s) {
      return (__builtin_amdgcn_sbfe(act, s, 1) & 0xFFFFu) | (__builtin_amdgcn_sbfe(act, s + 1, 1) & 0xFFFF0000u);
    };
    m0 = pair(0);
    m1 = pair(2);
    m2 = pair(4);
    m3 = pair(6);
  }
  hi = __builtin_bit_cast(f16x8, i32x4{(int)(H0 & m0), (int)(H1 & m1), (int)(H0 & m2), (int)(H1 & m3)});
  lo = __builtin_bit_cast(f16x8, i32x4{(int)(L0 & m0), (int)(L1 & m1), (int)(L0 & m2), (int)(L1 & m3)});
}

// kVec: O and I multiples of 4 and out, x 16-byte aligned (16-byte output stores and x
// loads); otherwise 4-byte ones.  kUniform: every knot row passed kan_knots_uniform.
//
// Split-K (nsplit > 1, for grids of fewer tiles than CUs): workgroup b computes split
// b % nsplit, feature groups [split*gper, split*gper + gper), of tile b / nsplit.  It
// writes its fp32 partial tile to `partial` and arrives on the tile's counter; the last
// of the tile's nsplit arrivals sums the partials in split order (so the result does not

// ---------------------------------------------------------------------------------------
// kan_fused: the warp-specialized GEMM.
//
// LDS (kLdsBytes):
//   weight ring, 3 x 32 KiB: hi then lo, 256 rows (output columns of the tile) x 64 B
//     (32 k) each, swizzle64
//   activation fragments, 2 x 16 KiB: [row block 0..7][hi, lo][lane] x 16 B, exactly the B
//     operand a consumer lane feeds its MFMA (one conflict-free 16-byte read)
//   the basis table of the groups in use, 32 KiB
//
// Chunk c of the workgroup's range is computed by the consumers from weight stage c % 3 and
// activation stage c % 2 while the producers write chunk c + 1's activations (evaluated in
// registers) and copy chunk c + 2's weight tile (direct-to-LDS), so copies have two chunks
// to land.  One workgroup barrier per chunk hands the stages over.  x is loaded one group
// ahead.  Spline chunk t of a group reads the table entries of its own features only (the
// features xb + t of the lanes), so once a chunk has been prepared its features' entries
// are refilled with the next group's, a step later.
// ---------------------------------------------------------------------------------------
// Chunk c's weight tile (rows n0 .. n0 + 255 of [q][Opad][32], hi and lo) into weight stage
// c % 3: one of the four copying waves (part) copies the 16-row groups 4 part .. 4 part + 3
// of each half.  A direct-to-LDS instruction writes 64 consecutive 16-byte slots (16 rows of
// 64 bytes); lane i fetches the chunk the swizzle places in slot i.  kPieces splits the 8
// copy instructions so a caller can interleave them with other work.
constexpr int kWeightCopies = 2 * (BN / 16) / 4;  // 1 KiB copies per copying wave per chunk
template <int kPiece, int kPieces>
__device__ __forceinline__ void copy_weight_tile(uint8_t* smem, __amdgpu_buffer_rsrc_t rhi, __amdgpu_buffer_rsrc_t rlo,
                                                 int q, int c, int Opad, int n0, int part, int lane) {
  uint8_t* st = smem + (c % kWStages) * kWStageBytes;
  const int r16 = lane / 4, logical = (lane % 4) ^ swz_w(r16);  // groups are 16-row aligned
  constexpr int kPer = kWeightCopies / 2 / kPieces;
#pragma unroll
  for (int i = kPiece * kPer; i < (kPiece + 1) * kPer; ++i) {
    const int group = part * (kWeightCopies / 2) + i;
    const unsigned off = (unsigned)(((size_t)q * Opad + n0 + group * 16 + r16) * 64 + 16 * logical);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rhi, (__attribute__((address_space(3))) void*)(st + group * 1024), 16, off, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rlo, (__attribute__((address_space(3))) void*)(st + kWHalfBytes + group * 1024), 16, off, 0, 0, 0);
  }
}

template <int kCp, bool kVec>
struct Producer {
  static constexpr int kQ = 1 + kCp;
  static constexpr int kX = kCp;                                    // x values per row block per group
  static constexpr int kCopies = kWeightCopies;
  static constexpr int kTableCopies = kTblBytes / 1024 / 4;         // 1 KiB table copies per producer wave
  static constexpr int kXLoads = kVec ? 2 * kX / 4 : 2 * kX;       // x load instructions per group
  static_assert(2 * kCopies + kTableCopies + kXLoads + 1 <= 63, "vmcnt holds at most 63");

  uint8_t* smem;
  __amdgpu_buffer_rsrc_t rhi, rlo, rx, rt;

  __device__ __forceinline__ void copy_weights(int c) const {
    copy_weight_tile<0, 1>(smem, rhi, rlo, (g0 + c / kQ) * kQ + c % kQ, c, Opad, n0, pw, lane);
  }

  // Piece kPiece of 4 of chunk c's weight copies (none past the last chunk).
  template <int kPiece>
  __device__ __forceinline__ void copy_weights_piece(int c) const {
    if (c < nchunks) copy_weight_tile<kPiece, 4>(smem, rhi, rlo, (g0 + c / kQ) * kQ + c % kQ, c, Opad, n0, pw, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
  int I, L, B, Opad, n0;
  int g0, nlg, nchunks;
  int lane, fr, fg, pw, xb;
  int row[2];      // this lane's batch rows (global) for its two row blocks
  bool uniform;    // every knot row is uniform: direct interval lookup
  int tgb;

  // Group lg's whole table into the table buffer: producer wave pw copies 1 KiB blocks
  // kTableCopies * pw .. +kTableCopies - 1; blocks past the group's table zero-fill.
  __device__ __forceinline__ void copy_table(int lg) const {
    uint8_t* dst = smem + kTblAt;
    const int g = g0 + lg;
#pragma unroll
    for (int i = 0; i < kTableCopies; ++i) {
      const int blk = pw * kTableCopies + i;
      const unsigned off = blk * 1024 < tgb ? (unsigned)((size_t)g * tgb + blk * 1024 + lane * 16) : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rt, (__attribute__((address_space(3))) void*)(dst + blk * 1024), 16, off, 0, 0, 0);
    }
  }

  // The entries of spline chunk t's features (t + kCp * m, m < 32 / kCp) of group lg into
  // the table buffer: producer wave pw < 32 / kCp copies feature t + kCp * pw, whose 64 L
  // bytes are 4 L lanes of one direct-to-LDS instruction.
  __device__ __forceinline__ void copy_table_slice(int lg, int t) const {
    if (lane < 4 * L) {
      const int fl = t + kCp * pw;
      const unsigned off = (unsigned)((size_t)(g0 + lg) * tgb + fl * 64 * L + lane * 16);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rt, (__attribute__((address_space(3))) void*)(smem + kTblAt + fl * 64 * L), 16, off, 0, 0, 0);
    }
  }

  // x at this lane's features xb .. xb + kX - 1 of group lg (past I or B: 0).
  __device__ __forceinline__ void load_x(int lg, float (&xs)[2][kX]) const {
    const int g = g0 + lg;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      if constexpr (kVec) {  // I % 4 == 0: a 4-feature run is wholly inside or past I
#pragma unroll
        for (int v = 0; v < kX / 4; ++v) {
          const int f = g * kGroup + xb + 4 * v;
          const unsigned off = (row[rb] < B && f < I) ? (unsigned)(((size_t)row[rb] * I + f) * 4) : kOutOfRange;
          const f32x4 val = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
#pragma unroll
          for (int e = 0; e < 4; ++e) xs[rb][4 * v + e] = val[e];
        }
      } else {
#pragma unroll
        for (int t = 0; t < kX; ++t) {
          const int f = g * kGroup + xb + t;
          const unsigned off = (row[rb] < B && f < I) ? (unsigned)(((size_t)row[rb] * I + f) * 4) : kOutOfRange;
          xs[rb][t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, off, 0, 0));
        }
      }
    }
  }

  // Chunk c's activations into stage c % 2: the lane's two row blocks evaluated, split and
  // stored as their MFMA fragments.  A silu chunk (kT < 0) takes slots 8 fg .. 8 fg + 7 from
  // the lane's x values 8 fg - xb ..; spline chunk kT expands feature xb + kT.
  // The weight copies of chunk cw are issued in four pieces between the parts of the
  // evaluation: a copy instruction holds the wave until the CU's memory pipeline takes it,
  // so spreading them lets the evaluation's VALU work fill that time.
  template <int kT>
  __device__ __forceinline__ void prepare_act(int c, const float (&xs)[2][kX], int cw, f32x2& k01next) const {
    uint8_t* act = smem + kActAt + (c & 1) * kActBytes;
    copy_weights_piece<0>(cw);
    // Both row blocks are evaluated before either is stored: a store to LDS orders every
    // later LDS read after it, so interleaving would serialise the two lookups.
    f16x8 hi[2], lo[2];
    if constexpr (kT < 0) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        float a[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          float xv = xs[rb][t];
          if constexpr (kX > 8) {
            // Both candidates as register values first: a select between two elements would
            // otherwise become a runtime index, which keeps the array in scratch memory.
            float xh = xs[rb][8 + t];
            asm volatile("" : "+v"(xv), "+v"(xh));
            xv = (fg & 1) ? xh : xv;
          }
          a[t] = silu(xv);
        }
        split8(a, hi[rb], lo[rb]);
        if (rb == 0) copy_weights_piece<1>(cw);
      }
      copy_weights_piece<2>(cw);
    } else {
      const float* fe = reinterpret_cast<const float*>(smem + kTblAt + (xb + kT) * 64 * L);
      TabFetch tf[2];
      if (uniform) {
        // The first two knots were read a step ago (k01); read the next spline chunk's now.
        const f32x2 k01 = k01next;
        k01next = *reinterpret_cast<const f32x2*>(smem + kTblAt + (xb + (kT + 1) % kX) * 64 * L);
        const float inv_h = __builtin_amdgcn_rcpf(k01.y - k01.x);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) tf[rb] = tab_locate_uniform(xs[rb][kT], k01.x, inv_h, fe, L);
      } else {
        f32x4 kn[4];
        tab_knots(fe, kn);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) tf[rb] = tab_locate_count(xs[rb][kT], kn, fe, L);
      }
      copy_weights_piece<1>(cw);
      tab_finish<kCp>(xs[0][kT], tf[0], (8 * fg) % kCp, hi[0], lo[0]);
      copy_weights_piece<2>(cw);
      tab_finish<kCp>(xs[1][kT], tf[1], (8 * fg) % kCp, hi[1], lo[1]);
    }
    copy_weights_piece<3>(cw);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int frag = 2 * pw + rb;
      *reinterpret_cast<f16x8*>(act + ((frag * 2 + 0) * 64 + lane) * 16) = hi[rb];
      *reinterpret_cast<f16x8*>(act + ((frag * 2 + 1) * 64 + lane) * 16) = lo[rb];
    }
  }

  // Step lg * kQ + kK runs while the consumers compute that chunk: it refills the entries
  // of the spline chunk prepared in the previous step with the next group's, loads the next
  // group's x at a group's first step, and writes the activations of chunk c = lg * kQ +
  // kK + 1 (spline chunk kK of group lg, or for kK = kQ - 1 the next group's silu chunk).
  // kLast: lg is the workgroup's last group.  Every condition is a constant, so
  // the compiler's own waits for x stay exact (a merge of paths would make it wait for
  // every load, the weight copies of the step included).
  template <bool kLast, int kK>
  __device__ __forceinline__ void step(int lg, float (&xcur)[2][kX], float (&xnext)[2][kX], f32x2& k01) const {
    const int c = lg * kQ + kK + 1;
    constexpr bool kCopyNext = !kLast || kK + 2 < kQ;   // chunk c + 1 exists
    constexpr bool kSlice = !kLast && kK >= 1;          // refill spline chunk kK - 1's entries
    constexpr bool kXNext = !kLast && kK == 0;
    // (only the waves with a feature of the slice issue its copy)
    const bool slice = kSlice && pw < kGroup / kCp;
    if (slice) copy_table_slice(lg + 1, kK - 1);
    if constexpr (kXNext) load_x(lg + 1, xnext);
    if constexpr (kK < kQ - 1) {
      prepare_act<kK>(c, xcur, c + 1, k01);
    } else if constexpr (!kLast) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int t = 0; t < kX; ++t) xcur[rb][t] = xnext[rb][t];
      prepare_act<-1>(c, xcur, c + 1, k01);
    } else {
      copy_weights_piece<0>(c + 1);  // past the last chunk: no copies
    }
    // Everything issued before this step (chunk c's weights among it) has landed.
    constexpr int kIssued = (kCopyNext ? kCopies : 0) + (kXNext ? kXLoads : 0);
    if (slice) wait_vmcnt<kIssued + 1>();
    else wait_vmcnt<kIssued>();
    barrier_no_vm_drain();
  }

  template <bool kLast, int... kKs>
  __device__ __forceinline__ void group_steps(int lg, float (&xcur)[2][kX], float (&xnext)[2][kX], f32x2& k01,
                                              std::integer_sequence<int, kKs...>) const {
    (step<kLast, kKs>(lg, xcur, xnext, k01), ...);
  }

  __device__ void run() const {
    float xcur[2][kX], xnext[2][kX];
    // Prologue: chunks 0 and 1's weights, the first group's table and x, chunk 0's
    // activations; the barrier after it publishes them.
    copy_weights(0);
    if (nchunks > 1) copy_weights(1);
    copy_table(0);
    load_x(0, xcur);
    wait_vmcnt<0>();
    f32x2 k01;
    prepare_act<-1>(0, xcur, nchunks, k01);  // (no copies: chunk 1's were issued above)
    barrier_no_vm_drain();
    // Spline chunk 0's first two knots: the whole table is visible after the barrier.
    k01 = *reinterpret_cast<const f32x2*>(smem + kTblAt + xb * 64 * L);
    // The steps of a group are unrolled, so every chunk kind is a constant.
    for (int lg = 0; lg + 1 < nlg; ++lg) group_steps<false>(lg, xcur, xnext, k01, std::make_integer_sequence<int, kQ>{});
    group_steps<true>(nlg - 1, xcur, xnext, k01, std::make_integer_sequence<int, kQ>{});
  }
};

// Consumer: chunk c's 96 MFMAs, two row blocks at a time and term-major, so an
// accumulator's next MFMA is 8 MFMAs behind its previous one (each accumulator sums
// hi*hi, lo*hi, hi*lo per chunk, in that order).  The next pair's activation fragments are
// read during a pair's MFMAs (one read per six MFMAs), so LDS reads overlap the MFMAs.
__device__ __forceinline__ void consume_chunk(const uint8_t* wst, const uint8_t* ast, int wave, int lane,
                                              f32x4 (&acc)[kRB][kCB]) {
  const int fr = lane % 16, fg = lane / 16;
  f16x8 wh[kCB], wl[kCB];
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb) {
    const int r = wave * (kCB * 16) + cb * 16 + fr;
    wh[cb] = __builtin_bit_cast(f16x8, *reinterpret_cast<const i32x4*>(wst + swizzle64(r, fg)));
    wl[cb] = __builtin_bit_cast(f16x8, *reinterpret_cast<const i32x4*>(wst + kWHalfBytes + swizzle64(r, fg)));
  }
  const uint8_t* act = ast + lane * 16;
  auto read_pair = [&](int rb, f16x8 (&ah)[2], f16x8 (&al)[2]) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      ah[r] = __builtin_bit_cast(f16x8, *reinterpret_cast<const i32x4*>(act + ((rb + r) * 2 + 0) * 1024));
      al[r] = __builtin_bit_cast(f16x8, *reinterpret_cast<const i32x4*>(act + ((rb + r) * 2 + 1) * 1024));
    }
  };
  f16x8 ah[2], al[2];
  read_pair(0, ah, al);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int rb = 0; rb < kRB; rb += 2) {
    f16x8 nh[2], nl[2];
    if (rb + 2 < kRB) read_pair(rb + 2, nh, nl);
#pragma unroll
    for (int term = 0; term < 3; ++term)
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb)
          acc[rb + r][cb] = mfma16(term == 1 ? wl[cb] : wh[cb], term == 2 ? al[r] : ah[r], acc[rb + r][cb]);
    if (rb + 2 < kRB) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);  // 6 MFMAs
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (rb + 2 < kRB) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        ah[r] = nh[r];
        al[r] = nl[r];
      }
    }
  }
}

// Output slot of a consumer accumulator: consumer wave wq, row block rb, column block cb,
// lane lq hold columns n0 + 64 wq + 16 cb + 4 (lq / 16) + 0..3 of batch row m0 + 16 rb +
// lq % 16, scaled back by the columns' scales.
__device__ __forceinline__ void store_slot(f32x4 val, int wq, int rb, int cb, int lq, int m0, int n0, int B, int O,
                                           const float* __restrict__ colscale, __amdgpu_buffer_rsrc_t ro, bool vec) {
  const int o = n0 + wq * (kCB * 16) + cb * 16 + 4 * (lq / 16);
  const int row = m0 + rb * 16 + lq % 16;
  val *= *reinterpret_cast<const f32x4*>(colscale + o);
  if (vec) {
    const unsigned off = (row < B && o < O) ? (unsigned)(((size_t)row * O + o) * 4) : kOutOfRange;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, val), ro, off, 0, 0);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const unsigned off = (row < B && o + e < O) ? (unsigned)(((size_t)row * O + o + e) * 4) : kOutOfRange;
      // Through a scalar: hipcc turned __builtin_bit_cast(unsigned, val[e]) into a store of
      // element 0 for every e.
      const float ve = val[e];
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ve), ro, off, 0, 0);
    }
  }
}

// Split-K handover, all 512 threads: after every consumer has written its partial, thread 0
// releases them at agent scope and arrives on the tile's counter; the tile's last arrival
// sums the nsplit partials of every slot in split order (so the result does not depend on
// which split arrives last), 16 slots per thread with each split's loads in flight
// together, resets the counter and writes the output.
template <bool kVec>
__device__ __forceinline__ void split_k_finish(uint8_t* smem, int tid, int split, int nsplit, int tile, int m0,
                                               int n0, int B, int O, const float* __restrict__ colscale,
                                               float* __restrict__ out, const float* __restrict__ partial,
                                               unsigned* __restrict__ counters) {
  __syncthreads();  // every consumer's partial stores have completed; the LDS stages are idle
  unsigned* flag = reinterpret_cast<unsigned*>(smem);
  if (tid == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const unsigned prev = __hip_atomic_fetch_add(counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev == (unsigned)nsplit - 1;
    if (last) __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  if (!*flag) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  constexpr int kSlots = BM * BN / 4;           // 16-byte slots per tile
  constexpr int kPer = kSlots / kThreads;       // per thread
  const int tiles = gridDim.x / nsplit;
  const size_t split_stride = (size_t)tiles * (BM * BN);
  const float* first = partial + (size_t)tile * (BM * BN);
  f32x4 sum[kPer];
  for (int sp = 0; sp < nsplit; ++sp) {
    f32x4 part[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u)
      part[u] = *reinterpret_cast<const f32x4*>(first + sp * split_stride + (size_t)(tid + u * kThreads) * 4);
#pragma unroll
    for (int u = 0; u < kPer; ++u) sum[u] = sp == 0 ? part[u] : sum[u] + part[u];
  }
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(out, (size_t)B * O * 4);
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int sl = tid + u * kThreads;  // = ((wq * kRB + rb) * kCB + cb) * 64 + lq
    const int lq = sl % kWave, cb = (sl / kWave) % kCB, rb = (sl / (kWave * kCB)) % kRB, wq = sl / (kWave * kCB * kRB);
    store_slot(sum[u], wq, rb, cb, lq, m0, n0, B, O, colscale, ro, kVec);
  }
}

// kVec: I and O multiples of 4, x and out 16-byte aligned (16-byte loads and stores);
// otherwise 4-byte ones.
//
// Split-K (nsplit > 1, for grids of fewer tiles than CUs): workgroup b computes split
// b % nsplit, feature groups [split*gper, split*gper + gper), of tile b / nsplit.  It
// writes its fp32 partial tile to `partial` and arrives on the tile's counter; the last
// of the tile's nsplit arrivals sums the partials in split order (so the result does not
// depend on which arrives last) and writes the output.
template <int kCp, bool kVec>
__global__ __launch_bounds__(kThreads) void kan_fused(
    const float* __restrict__ x, const float* __restrict__ tables, const int* __restrict__ uflags, int nflags,
    int B, int I, int O, int L, int ngroups, int Opad, const _Float16* __restrict__ bhi,
    const _Float16* __restrict__ blo, const float* __restrict__ colscale, float* __restrict__ out, int nsplit,
    int gper, float* __restrict__ partial, unsigned* __restrict__ counters) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int kQ = 1 + kCp;
  const int tm = (B + BM - 1) / BM, tn = Opad / BN;
  const int split = blockIdx.x % nsplit, tile = blockIdx.x / nsplit;
  const int g0 = split * gper, g1 = min(ngroups, g0 + gper);
  const int nchunks = (g1 - g0) * kQ;
  int mt, nt;
  tile_of(tile, tm, tn, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);

  if (wave >= kConsumerWaves) {
    {
      Producer<kCp, kVec> p;
      p.smem = smem;
      p.I = I; p.L = L; p.B = B; p.Opad = Opad; p.n0 = n0;
      p.g0 = g0; p.nlg = g1 - g0; p.nchunks = nchunks;
      p.lane = lane; p.fr = lane % 16; p.fg = lane / 16; p.pw = wave - kConsumerWaves;
      p.xb = ((8 * p.fg) / kCp) * kCp;
      p.row[0] = m0 + 32 * p.pw + p.fr;
      p.row[1] = p.row[0] + 16;
      p.tgb = tbl_group_bytes(L);
      const size_t wbytes = (size_t)ngroups * kQ * Opad * kChunk * 2;
      p.rhi = make_rsrc(bhi, wbytes);
      p.rlo = make_rsrc(blo, wbytes);
      p.rx = make_rsrc(x, (size_t)B * I * 4);
      p.rt = make_rsrc(tables, (size_t)ngroups * p.tgb);
      bool ok = true;
      for (int i = lane; i < nflags; i += kWave) ok = ok && uflags[i] != 0;
      p.uniform = __builtin_amdgcn_ballot_w64(!ok) == 0;
      p.run();
    }
    wait_vmcnt<0>();  // no copy may still be writing LDS past this point
    if (nsplit > 1) split_k_finish<kVec>(smem, tid, split, nsplit, tile, m0, n0, B, O, colscale, out, partial, counters);
    return;
  }

  f32x4 acc[kRB][kCB];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  barrier_no_vm_drain();  // stage 0 is ready
  for (int c = 0; c < nchunks; ++c) {
    consume_chunk(smem + (c % kWStages) * kWStageBytes, smem + kActAt + (c & 1) * kActBytes, wave, lane, acc);
    barrier_no_vm_drain();
  }

  if (nsplit > 1) {
    // This thread's 16-byte slots of the partial tile: (wave, rb, cb, lane), so every
    // store instruction of a wave covers 1 KiB of contiguous memory.
    const int tiles = gridDim.x / nsplit;
    float* mine = partial + ((size_t)split * tiles + tile) * (BM * BN);
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb)
        *reinterpret_cast<f32x4*>(mine + (((wave * kRB + rb) * kCB + cb) * kWave + lane) * 4) = acc[rb][cb];
    split_k_finish<kVec>(smem, tid, split, nsplit, tile, m0, n0, B, O, colscale, out, partial, counters);
    return;
  }

  // Epilogue.
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(out, (size_t)B * O * 4);
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) store_slot(acc[rb][cb], wave, rb, cb, lane, m0, n0, B, O, colscale, ro, kVec);
}

}  // namespace kan
}  // namespace taskops
