// efficient_kan kernels for gfx950 (instantiated by efficient_kan.hip).
//
// Op: tasks/efficient_kan/reference.py:33-51 (fp64 oracle :54-57):
//   out[b,o] = sum_i silu(x[b,i]) Wb[o,i] + sum_i sum_c B_c(x[b,i]) Ws[o,i,c] sc[o,i]
// with B_c the order-p B-spline bases on feature i's knot row (Cox-de Boor).
//
// One contraction over K = I * (1 + C') (C' = C rounded up to 8, 16 or 32) on the fp16
// MFMA v_mfma_f32_16x16x32_f16 with a three-term split for fp32-level accuracy: every
// operand v is carried as hi = fp16(v) and lo = fp16(v - hi), and each product as
// hi*hi + hi*lo + lo*hi (the dropped lo*lo term is ~2^-22 relative), accumulated in fp32.
//
// K order: features in groups of 32; each group is one "silu" chunk (32 features, k =
// feature) followed by C' "spline" chunks; spline chunk t holds the C' bases of the 32/C'
// features i*C' + t (k = i*C' + basis).  In MFMA layout lane l supplies k = 8*(l/16) .. +7
// of batch row l % 16, so over one group a lane needs x at one contiguous run of C'
// features, and in a spline chunk it owns one (row, feature) and 8 of its bases: it finds
// x's knot interval, evaluates the four bases nonzero there from per-interval cubic
// coefficients and shifts them into its 8 slots, straight in registers — the expanded
// activations never touch LDS or HBM.
//
// Per call, kan_prepare and kan_pack (a) write the weights ([Wb | Ws*sc], the A operand)
// in that K order as fp16 hi/lo with a per-output-column power-of-two scale (so neither
// half under- or overflows) and (b) tabulate each feature's knot row and per-interval
// basis cubics.
// The GEMM streams the weights through an LDS ring with direct-to-LDS loads, copies each
// feature group's table into LDS, and undoes the column scale in the epilogue.
#pragma once

#include "common.hpp"

namespace taskops {
namespace kan {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;     // 4 waves, one per SIMD
constexpr int kWaves = kThreads / 64;
constexpr int BM = 128;           // batch rows per workgroup: 32 per wave = 2 row blocks
constexpr int BN = 256;           // output columns per workgroup: 16 column blocks
constexpr int kNJ = BN / 16;
constexpr int kGroup = 32;        // features per group
constexpr int kChunk = 32;        // k per MFMA chunk
constexpr int kMaxKnots = 16;     // fast path: grid_size + 2*order + 1 <= 16
constexpr int kOrder = 3;         // the fast path's spline order
constexpr int kTileBytes = BN * kChunk * 2;          // one half (hi or lo) of a chunk tile: 16 KiB
constexpr int kStageBytes = 2 * kTileBytes;          // hi + lo: 32 KiB
constexpr int kGroupsPerWave = BN / 16 / kWaves;     // 16-row tile groups each wave copies
constexpr int kRawBufferFlags = 0x00020000;
constexpr unsigned kOutOfRange = 0x80000000u;

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
constexpr int kTblBytes = 32 * 1024;  // LDS table buffer: 32 features * 64 * L bytes, L <= 16

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
// Weight preparation, in two launches: kan_prepare finds each output column's scale,
// kan_pack writes the GEMM's A operand and builds the basis tables.
// bhi/blo: [nchunks][Opad][32] fp16; chunk q = g*(1+Cp) + sub; sub 0 holds Wb[o, 32g + s],
// sub >= 1 holds (Ws*sc)[o, f, c] with f = 32g + (s/Cp)*Cp + (sub-1), c = s % Cp (zero
// past I, O or C), all times 2^e.  So over a group's spline chunks the lanes that supply
// slots s..s+7 of a chunk walk the features (s/Cp)*Cp .. +Cp-1: the same 8 (Cp = 8) or 16
// features whose silu values they supply, and the GEMM loads each lane's x values as one
// contiguous run.  colscale[o] = 2^-e with e chosen so max|column| * 2^e is in
// [2^14, 2^15), so neither fp16 half under- or overflows.
// ---------------------------------------------------------------------------------------
// kan_prepare: workgroup o reduces column o (contiguous rows of wb, sc and ws) to
// colscale[o].  Workgroup 0 also zeroes kan_gemm's split-K arrival counters (their place in
// the workspace moves with the shape, so every call starts them from zero).
__global__ __launch_bounds__(256) void kan_prepare(
    const float* __restrict__ wb, const float* __restrict__ ws, const float* __restrict__ sc, int I,
    int O, int C, float* __restrict__ colscale, unsigned* __restrict__ counters, int ncounters) {
  __shared__ float red[4];
  const int o = blockIdx.x;
  if (o == 0)
    for (int i = threadIdx.x; i < ncounters; i += 256) counters[i] = 0u;
  float mx = 0.0f;
  if (o < O) {
    // max_c |ws * s| = |s| * max_c |ws| exactly (rounding is monotonic).  Features are
    // unrolled four at a time so each thread keeps its loads in flight together.
    const float* wsc = ws + (size_t)o * I * C;
    const bool vec = C % 4 == 0 && (reinterpret_cast<uintptr_t>(wsc) & 15) == 0;
    for (int i0 = threadIdx.x; i0 < I; i0 += 4 * 256) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * 256;
        if (i < I) {
          float m = 0.0f;
          if (vec) {
            for (int c = 0; c < C; c += 4) {
              const f32x4 v = *reinterpret_cast<const f32x4*>(wsc + (size_t)i * C + c);
              m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
          } else {
            for (int c = 0; c < C; ++c) m = fmaxf(m, fabsf(wsc[(size_t)i * C + c]));
          }
          mx = fmaxf(mx, fmaxf(fabsf(wb[(size_t)o * I + i]), fabsf(sc[(size_t)o * I + i]) * m));
        }
      }
    }
  }
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (mx > 0.0f && mx < __builtin_inff()) e = 14 - ilogbf(mx);
  e = e > 100 ? 100 : (e < -100 ? -100 : e);
  if (threadIdx.x == 0) colscale[o] = ldexpf(1.0f, -e);
}

// Basis tables, one thread per table entry (L per feature: the knot row and the L - 1
// intervals); uflags[block] = 1 when every knot row the block wrote is uniform
// (kan_knots_uniform), else 0.
__device__ __forceinline__ void kan_tables_block(int block, const float* __restrict__ grid, int I, int L,
                                                 int ngroups, float* __restrict__ tables,
                                                 int* __restrict__ uflags) {
  const int idx = block * 256 + (int)threadIdx.x;
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
// need nothing from the packing, so they run beside it.  Workgroup tblocks + ct + g *
// (Opad / 8) writes the 1 + Cp chunks of feature group g for columns 8ct .. 8ct+7; thread
// (column o, feature fl) writes all of its feature's bases, which
// form one run of Cp slots (fl / Cp) * Cp .. in spline chunk 1 + fl % Cp, and threads
// fl < 4 also write silu slots 8 fl .. +7.  A column's 32 threads so read its contiguous
// ws rows, and the four threads that fill one 64-byte chunk row sit in the same wave.
constexpr int kPackCols = 8;
template <int kCp>
__global__ __launch_bounds__(256) void kan_pack(
    const float* __restrict__ wb, const float* __restrict__ ws, const float* __restrict__ sc, int I,
    int O, int C, int Opad, const float* __restrict__ colscale, _Float16* __restrict__ bhi,
    _Float16* __restrict__ blo, const float* __restrict__ grid, int L, int ngroups, int tblocks,
    float* __restrict__ tables, int* __restrict__ uflags) {
  static_assert(kCp % 8 == 0 && kPackCols * kGroup == 256, "thread per (column, feature)");
  if ((int)blockIdx.x < tblocks) {
    kan_tables_block(blockIdx.x, grid, I, L, ngroups, tables, uflags);
    return;
  }
  constexpr int kSub = 1 + kCp;
  const int b = (int)blockIdx.x - tblocks, ntiles = Opad / kPackCols;
  const int g = b / ntiles, oc = (int)threadIdx.x / kGroup, fl = (int)threadIdx.x % kGroup;
  const int o = (b % ntiles) * kPackCols + oc, f = g * kGroup + fl;
  const float scale = 1.0f / colscale[o];  // 2^e, exact
  auto put = [&](int sub, int slot, const float* v) {
    f16x8 h8, l8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float w = v[e] * scale;
      const _Float16 h = (_Float16)w;
      h8[e] = h;
      l8[e] = (_Float16)(w - (float)h);
    }
    const size_t dst = ((size_t)(g * kSub + sub) * Opad + o) * kChunk + slot;
    *reinterpret_cast<f16x8*>(bhi + dst) = h8;
    *reinterpret_cast<f16x8*>(blo + dst) = l8;
  };
  float v[kCp];
#pragma unroll
  for (int c = 0; c < kCp; ++c) v[c] = 0.0f;
  if (o < O && f < I) {
    const float s = sc[(size_t)o * I + f];
    const float* row = ws + ((size_t)o * I + f) * C;
    if (C % 4 == 0 && (reinterpret_cast<uintptr_t>(ws) & 15) == 0) {
#pragma unroll
      for (int c4 = 0; c4 < kCp / 4; ++c4) {
        if (4 * c4 < C) {
          const f32x4 q = *reinterpret_cast<const f32x4*>(row + 4 * c4);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * c4 + e] = q[e] * s;
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < kCp; ++c)
        if (c < C) v[c] = row[c] * s;
    }
  }
#pragma unroll
  for (int h = 0; h < kCp / 8; ++h) put(1 + fl % kCp, (fl / kCp) * kCp + 8 * h, v + 8 * h);
  if (fl < 4) {
    float u[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int f2 = g * kGroup + 8 * fl + e;
      u[e] = o < O && f2 < I ? wb[(size_t)o * I + f2] : 0.0f;
    }
    put(0, 8 * fl, u);
  }
}

// ---------------------------------------------------------------------------------------
// GEMM with the fused activation expansion.
//
// 128x256 output tile per workgroup of 4 waves (one per SIMD); wave w owns batch rows
// 32w..32w+31 (2 row blocks) x all 256 columns (16 column blocks, 128 fp32 accumulators in
// AGPRs).  Weights stream through a 4-stage LDS ring of 32 KiB chunks (32 k x 256 columns,
// hi then lo) filled by direct-to-LDS copies three chunks ahead; the group's table
// (knots + cubics, <= 32 KiB) has one LDS buffer, copied at the previous group's last
// chunk — when that group's last spline chunk has been expanded — before that chunk's
// weight copy, so the group's first chunk waits for it.  x values are prefetched into
// registers one group ahead.
//
// The activations of chunk q+1 are built during chunk q's MFMAs.  A wave issues its MFMAs
// in order and cannot pass an outstanding wait, so each chunk runs in four quarters of 24
// MFMAs (4 column blocks, weight fragments read a quarter ahead): the next chunk's knot
// rows are read before Q1, whose MFMAs cover that latency; the interval lookup is
// interleaved with Q2's MFMAs and issues the coefficient reads, which the rest of Q2
// covers; the cubic evaluation, split and slot routing of row block 0 are interleaved
// with Q3's MFMAs and those of row block 1 with Q4's.  The loop body is
// one whole feature group unrolled (every chunk kind and wait count is a constant) and
// weight and table copies past the end zero-fill through the buffer descriptors, so no
// branch surrounds the MFMAs (which would make the compiler copy the accumulators).
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

// Copy part `part` (0 .. kGroupsPerWave-1) of this wave's share of chunk q's hi and lo
// tiles (rows n0..n0+BN-1 of [q][Opad][32]) into an LDS stage: one 16-row group of each
// half.  A direct-to-LDS instruction writes 64 consecutive 16-byte slots (16 rows of 64
// bytes); lane i fetches the chunk the swizzle places in slot i.
__device__ __forceinline__ void dma_chunk_part(__amdgpu_buffer_rsrc_t rhi, __amdgpu_buffer_rsrc_t rlo,
                                               uint8_t* stage, int q, int Opad, int n0, int wave,
                                               int lane, int part) {
  const int r16 = lane / 4, logical = (lane % 4) ^ swz_w(r16);  // groups are 16-row aligned
  static_assert(kGroupsPerWave * kWaves * 16 == BN, "tile rows split evenly over waves");
  const int group = wave * kGroupsPerWave + part;
  const int row = group * 16 + r16;
  const unsigned off = (unsigned)(((size_t)q * Opad + n0 + row) * 64 + 16 * logical);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rhi, (__attribute__((address_space(3))) void*)(stage + group * 1024), 16, off, 0, 0, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rlo, (__attribute__((address_space(3))) void*)(stage + kTileBytes + group * 1024), 16, off,
      0, 0, 0);
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
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
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
  const f16x2 l01 = __builtin_convertvector(f32x2{N[0] - (float)h01.x, N[1] - (float)h01.y}, f16x2);
  const f16x2 l23 = __builtin_convertvector(f32x2{N[2] - (float)h23.x, N[3] - (float)h23.y}, f16x2);
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
// depend on which arrives last) and writes the output.
template <int kCp, bool kVec, bool kUniform>
__device__ __forceinline__ void kan_gemm_body(
    uint8_t* smem, const float* __restrict__ x, const float* __restrict__ tables, int B, int I, int O,
    int L, int ngroups, int Opad, const _Float16* __restrict__ bhi, const _Float16* __restrict__ blo,
    const float* __restrict__ colscale, float* __restrict__ out, int nsplit, int gper,
    float* __restrict__ partial, unsigned* __restrict__ counters) {
  constexpr int kStages = 4;
  constexpr int kQ = 1 + kCp;                        // chunks per feature group
  constexpr int kPerStep = 2 * kGroupsPerWave;        // weight copy instructions per wave per chunk
  constexpr int kX = kCp;                             // x values per lane and row block per group
  uint8_t* tbl = smem + kStages * kStageBytes;
  const int tm = (B + BM - 1) / BM, tn = Opad / BN;
  const int split = blockIdx.x % nsplit, tile = blockIdx.x / nsplit;
  const int g0 = split * gper, g1 = min(ngroups, g0 + gper);
  int mt, nt;
  tile_of(tile, tm, tn, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int nq = ngroups * kQ;
  const size_t tile_bytes = (size_t)nq * Opad * kChunk * 2;
  const __amdgpu_buffer_rsrc_t rhi = make_rsrc(bhi, tile_bytes);
  const __amdgpu_buffer_rsrc_t rlo = make_rsrc(blo, tile_bytes);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (size_t)B * I * 4);
  const int tgb = tbl_group_bytes(L), tper = tgb / 4096;  // 1 KiB table copies per wave per group
  const __amdgpu_buffer_rsrc_t rt = make_rsrc(tables, (size_t)ngroups * tgb);
  const int fr = lane % 16, fg = lane / 16;
  const int row0 = m0 + wave * 32;

  f32x4 acc[2][kNJ];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int j = 0; j < kNJ; ++j) acc[rb][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // This lane's features within a group are xb .. xb + kX - 1 (slot t = feature xb + t):
  // spline chunk t expands feature xb + t, and the silu chunk's features 8*fg .. +7 are
  // slots 8*fg - xb .. +7.
  const int xb = ((8 * fg) / kCp) * kCp;
  float xcur[2][kX], xnext[2][kX];
  auto prefetch = [&](int g) {  // past I or B: reads as 0 (against zero weights)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int row = row0 + rb * 16 + fr;
      if constexpr (kVec) {  // I % 4 == 0: a 4-feature run is wholly inside or past I
#pragma unroll
        for (int v = 0; v < kX / 4; ++v) {
          const int f = g * kGroup + xb + 4 * v;
          const unsigned off = (row < B && f < I) ? (unsigned)((row * I + f) * 4) : kOutOfRange;
          const f32x4 val = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
#pragma unroll
          for (int e = 0; e < 4; ++e) xnext[rb][4 * v + e] = val[e];
        }
      } else {
#pragma unroll
        for (int t = 0; t < kX; ++t) {
          const int f = g * kGroup + xb + t;
          const unsigned off = (row < B && f < I) ? (unsigned)((row * I + f) * 4) : kOutOfRange;
          xnext[rb][t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, off, 0, 0));
        }
      }
    }
  };
  auto dma_part = [&](int q, int part) {
    dma_chunk_part(rhi, rlo, smem + (q % kStages) * kStageBytes, q, Opad, n0, wave, lane, part);
  };
  auto dma = [&](int q) {
#pragma unroll
    for (int i = 0; i < kGroupsPerWave; ++i) dma_part(q, i);
  };
  auto dma_table = [&](int g) {
    for (int i = 0; i < tper; ++i) {
      const int blk = wave * tper + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rt, (__attribute__((address_space(3))) void*)(tbl + blk * 1024), 16,
          (unsigned)(g * tgb + blk * 1024 + lane * 16), 0, 0, 0);
    }
  };
  auto silu_rb = [&](const float (&xs)[2][kX], int rb, f16x8& hi, f16x8& lo) {
    float v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      float xv = xs[rb][t];
      if constexpr (kX > 8) xv = (fg & 1) ? xs[rb][8 + t] : xv;  // slot 8*fg - xb + t
      v[t] = silu(xv);
    }
    split8(v, hi, lo);
  };
  auto silu_chunk = [&](const float (&xs)[2][kX], f16x8 (&hi)[2], f16x8 (&lo)[2]) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) silu_rb(xs, rb, hi[rb], lo[rb]);
  };
  // Row block rb's activations for the next chunk (a spline chunk from this group's table,
  // or the next group's silu chunk).
  auto expand_rb = [&](bool spline_next, int xs, const TabFetch& tf, int rb, f16x8& hi, f16x8& lo) {
    if (spline_next)
      tab_finish<kCp>(xcur[rb][xs], tf, (8 * fg) % kCp, hi, lo);
    else
      silu_rb(xnext, rb, hi, lo);
  };

  // Prologue: group g0's table, its first 3 weight chunks, its x, its silu activations.
  dma_table(g0);
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) dma(g0 * kQ + s);
  prefetch(g0);
  f16x8 ahi[2], alo[2];
  {
    float x0[2][kX];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int t = 0; t < kX; ++t) x0[rb][t] = xnext[rb][t];
    silu_chunk(x0, ahi, alo);
  }

  constexpr int kXLoads = kVec ? 2 * kX / 4 : 2 * kX;  // x load instructions per group
  // vmcnt counts to 63; a smaller allowance only waits for more of the later loads.
  constexpr int kW0 = kPerStep + kXLoads > 63 ? 63 : kPerStep + kXLoads;
  constexpr int kW12 = 2 * kPerStep + kXLoads > 63 ? 63 : 2 * kPerStep + kXLoads;
  for (int g = g0; g < g1; ++g) {
    barrier_no_vm_drain();
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int t = 0; t < kX; ++t) xcur[rb][t] = xnext[rb][t];
    prefetch(g + 1);
#pragma unroll
    for (int k = 0; k < kQ; ++k) {
      const int q = g * kQ + k;
      // Issue order: the table of group g and chunk q0+2 at the previous group's last
      // chunk, the x prefetch at group start, chunk q+3 at chunk q.  Chunk q (and at k == 0
      // the table) has landed once at most these later ones are outstanding.
      if (k == 0) wait_vmcnt<kW0>();
      else if (k <= 2) wait_vmcnt<kW12>();
      else wait_vmcnt<2 * kPerStep>();
      barrier_no_vm_drain();
      if (k == kQ - 1) dma_table(g + 1);
      // Chunk q+3 goes to the stage chunk q-1 used, which every wave has finished reading
      // (barrier above).  Its copies are issued a part per quarter: issued together, the
      // workgroup's 32 copy instructions queue at the memory pipeline and hold up the
      // waves' MFMAs behind them.
      static_assert(kGroupsPerWave == 4, "one copy part per quarter");
      dma_part(q + kStages - 1, 0);

      const uint8_t* st = smem + (q % kStages) * kStageBytes;
      f16x8 wa[4][2], wb[4][2];
      auto load_w = [&](int j0, f16x8 (&w)[4][2]) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int r = (j0 + u) * 16 + fr;
          w[u][0] = __builtin_bit_cast(f16x8, *reinterpret_cast<const i32x4*>(st + swizzle64(r, fg)));
          w[u][1] = __builtin_bit_cast(f16x8, *reinterpret_cast<const i32x4*>(st + kTileBytes + swizzle64(r, fg)));
        }
      };
      // 4 column blocks x 2 row blocks x 3 split terms; weights are the A operand, so a
      // block is [o][b] (lane: batch row fr, registers: 4 consecutive columns).  Issued
      // term by term over the 8 blocks, so an accumulator's next MFMA is 8 MFMAs behind
      // its previous one (each accumulator still sums hi*hi, lo*hi, hi*lo in that order).
      auto mfma_w = [&](int j0, const f16x8 (&w)[4][2]) {
#pragma unroll
        for (int term = 0; term < 3; ++term)
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
              acc[rb][j0 + u] = mfma16(term == 1 ? w[u][1] : w[u][0], term == 2 ? alo[rb] : ahi[rb], acc[rb][j0 + u]);
      };
      // The next chunk: this group's spline chunk k+1, or the next group's silu chunk.
      const bool spline_next = k + 1 < kQ;
      const int fl = spline_next ? xb + k : 0;  // feature in group
      const float* fe = reinterpret_cast<const float*>(tbl + fl * 64 * L);
      const int xs = spline_next ? k : 0;
      f16x8 nhi[2], nlo[2];
      f32x4 kn[4];
      f32x2 k01;
      TabFetch tf[2];
      load_w(0, wa);
      if (spline_next) {
        if constexpr (kUniform) k01 = *reinterpret_cast<const f32x2*>(fe);
        else tab_knots(fe, kn);
      }
      __builtin_amdgcn_sched_barrier(0);
      mfma_w(0, wa);  // Q1
      load_w(4, wb);
      __builtin_amdgcn_sched_barrier(0);
      dma_part(q + kStages - 1, 1);
      if (spline_next) {
        if constexpr (kUniform) {
          const float inv_h = __builtin_amdgcn_rcpf(k01.y - k01.x);
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) tf[rb] = tab_locate_uniform(xcur[rb][xs], k01.x, inv_h, fe, L);
        } else {
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) tf[rb] = tab_locate_count(xcur[rb][xs], kn, fe, L);
        }
      }
      mfma_w(4, wb);  // Q2, interleaved with the interval lookup, which issues the coefficient reads
      load_w(8, wa);
#pragma unroll
      for (int u = 0; u < 24; ++u) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // 2 VALU
      }
      __builtin_amdgcn_sched_barrier(0);
      dma_part(q + kStages - 1, 2);
      expand_rb(spline_next, xs, tf[0], 0, nhi[0], nlo[0]);
      mfma_w(8, wa);  // Q3, interleaved with row block 0's evaluation
      load_w(12, wb);
#pragma unroll
      for (int u = 0; u < 24; ++u) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // 3 VALU
      }
      __builtin_amdgcn_sched_barrier(0);
      dma_part(q + kStages - 1, 3);
      expand_rb(spline_next, xs, tf[1], 1, nhi[1], nlo[1]);
      mfma_w(12, wb);  // Q4, interleaved with row block 1's
#pragma unroll
      for (int u = 0; u < 24; ++u) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // 3 VALU
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        ahi[rb] = nhi[rb];
        alo[rb] = nlo[rb];
      }
    }
  }
  wait_vmcnt<0>();  // no copy may still be writing LDS when the workgroup exits

  if (nsplit > 1) {
    // This thread's 16-byte slots of the tile: (wave, rb, j, lane), so every store and
    // load instruction of a wave covers 1 KiB of contiguous memory.
    constexpr int kTileFloats = BM * BN;
    auto slot = [&](int rb, int j) { return (((wave * 2 + rb) * kNJ + j) * kWave + lane) * 4; };
    const int tiles = gridDim.x / nsplit;
    float* mine = partial + ((size_t)split * tiles + tile) * kTileFloats;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int j = 0; j < kNJ; ++j) *reinterpret_cast<f32x4*>(mine + slot(rb, j)) = acc[rb][j];
    __syncthreads();  // every wave's stores have completed to L2; the LDS ring is idle
    unsigned* flag = reinterpret_cast<unsigned*>(smem);
    if (tid == 0) {
      // Release at agent scope (writes the partial back past this XCD's L2), then arrive.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      const unsigned prev = __hip_atomic_fetch_add(counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *flag = prev == (unsigned)nsplit - 1;
    }
    __syncthreads();
    if (!*flag) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const size_t split_stride = (size_t)tiles * kTileFloats;
    const float* first = partial + (size_t)tile * kTileFloats;
    // Split by split, all 32 of the thread's slots at once, so the loads of a split are in
    // flight together; each slot sums splits 0, 1, ... in order, this workgroup's own split
    // from its registers.
    f32x4 own[2][kNJ];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int j = 0; j < kNJ; ++j) own[rb][j] = acc[rb][j];
    for (int sp = 0; sp < nsplit; ++sp) {
      const float* src = first + sp * split_stride;
      f32x4 part[2][kNJ];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int j = 0; j < kNJ; ++j)
          part[rb][j] = sp == split ? own[rb][j] : *reinterpret_cast<const f32x4*>(src + slot(rb, j));
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int j = 0; j < kNJ; ++j) acc[rb][j] = sp == 0 ? part[rb][j] : acc[rb][j] + part[rb][j];
    }
  }

  // Epilogue: lane holds columns n0 + 16j + 4*fg + 0..3 of batch row row0 + 16rb + fr.
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(out, (size_t)B * O * 4);
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    const int o = n0 + j * 16 + 4 * fg;
    const f32x4 cs = *reinterpret_cast<const f32x4*>(colscale + o);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int row = row0 + rb * 16 + fr;
      const f32x4 val = acc[rb][j] * cs;
      if constexpr (kVec) {
        const unsigned off = (row < B && o < O) ? (unsigned)((row * O + o) * 4) : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, val), ro, off, 0, 0);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const unsigned off = (row < B && o + e < O) ? (unsigned)((row * O + o + e) * 4) : kOutOfRange;
          // Through a scalar: hipcc turned __builtin_bit_cast(unsigned, val[e]) into a store of
          // element 0 for every e.
          const float ve = val[e];
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ve), ro, off, 0, 0);
        }
      }
    }
  }
}

// The uniform-grid flags (one per table workgroup of kan_prepare) are read once; the branch
// selects one of two whole loop bodies, so no branch sits inside the MFMA loop.
template <int kCp, bool kVec>
__global__ __launch_bounds__(kThreads) void kan_gemm(
    const float* __restrict__ x, const float* __restrict__ tables, const int* __restrict__ uflags,
    int nflags, int B, int I, int O, int L, int ngroups, int Opad, const _Float16* __restrict__ bhi,
    const _Float16* __restrict__ blo, const float* __restrict__ colscale, float* __restrict__ out, int nsplit,
    int gper, float* __restrict__ partial, unsigned* __restrict__ counters) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  bool ok = true;
  for (int i = (int)threadIdx.x % kWave; i < nflags; i += kWave) ok = ok && uflags[i] != 0;
  if (__builtin_amdgcn_ballot_w64(!ok) == 0)
    kan_gemm_body<kCp, kVec, true>(smem, x, tables, B, I, O, L, ngroups, Opad, bhi, blo, colscale, out, nsplit,
                                   gper, partial, counters);
  else
    kan_gemm_body<kCp, kVec, false>(smem, x, tables, B, I, O, L, ngroups, Opad, bhi, blo, colscale, out, nsplit,
                                    gper, partial, counters);
}

}  // namespace kan
}  // namespace taskops
