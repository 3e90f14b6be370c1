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
// feature) followed by C' "spline" chunks (32/C' features x C' bases, k = feature*C' +
// basis).  In MFMA layout lane l supplies k = 8*(l/16) .. +7 of batch row l % 16, so in
// a spline chunk each lane owns one (row, feature) and 8 of its bases: it finds x's knot
// interval, evaluates the four bases nonzero there from per-interval cubic coefficients
// and shifts them into its 8 slots, straight in registers — the expanded activations
// never touch LDS or HBM.
//
// Per call, kan_prepare (a) writes the weights ([Wb | Ws*sc], the A operand) in that K
// order as fp16 hi/lo with a per-output-column power-of-two scale (so neither half under-
// or overflows) and (b) tabulates each feature's knot row and per-interval basis cubics.
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
// are nonzero on [t_j, t_{j+1}), as polynomials in u = x - t_j (16 floats: basis r's c0..c3
// at [4r, 4r+4)).  A basis outside [0, C) has zero coefficients.  The polynomials come
// from the Cox-de Boor recursion carried out on polynomials in fp64 with the reference's
// index ranges (tasks/efficient_kan/reference.py:33-39: N_{k,p} exists for 0 <= k <=
// L-2-p); a zero-width knot span contributes nothing.  Layout: [group][tbl_group_bytes],
// feature fl of a group at fl * 64 * L bytes, so one group is one contiguous copy.
// ---------------------------------------------------------------------------------------
constexpr int kTblBytes = 32 * 1024;  // LDS table buffer: 32 features * 64 * L bytes, L <= 16

__host__ __device__ inline int tbl_group_bytes(int L) { return 4096 * ((L + 1) / 2); }

__host__ __device__ void kan_table_feature(const float* __restrict__ knots_row, int L, float* __restrict__ dst) {
  double t[kMaxKnots];
  for (int k = 0; k < kMaxKnots; ++k) t[k] = k < L ? (double)knots_row[k] : 0.0;
  for (int k = 0; k < kMaxKnots; ++k) dst[k] = k < L ? knots_row[k] : __builtin_inff();
  for (int j = 0; j + 1 < L; ++j) {
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
    for (int r = 0; r <= kOrder; ++r)
      for (int c = 0; c < 4; ++c) dst[kMaxKnots + j * 16 + 4 * r + c] = (float)P[r][c];
  }
}

// ---------------------------------------------------------------------------------------
// Weight preparation: one workgroup per output column o.
// bhi/blo: [nchunks][Opad][32] fp16; chunk q = g*(1+Cp) + sub; sub 0 holds Wb[o, 32g + s],
// sub >= 1 holds (Ws*sc)[o, f, c] with f = 32g + (sub-1)*(32/Cp) + s/Cp, c = s % Cp
// (zero past I or C).  colscale[o] = 2^-e with e chosen so max|column| * 2^e is in
// [2^14, 2^15).
// ---------------------------------------------------------------------------------------
// Workgroups past Opad build the basis tables instead (one feature per thread), when
// `tables` is given.
__global__ __launch_bounds__(256) void kan_prepare(
    const float* __restrict__ wb, const float* __restrict__ ws, const float* __restrict__ sc, int I,
    int O, int C, int Cp, int ngroups, int Opad, _Float16* __restrict__ bhi,
    _Float16* __restrict__ blo, float* __restrict__ colscale, const float* __restrict__ grid = nullptr,
    int L = 0, float* __restrict__ tables = nullptr) {
  __shared__ float red[4];
  if ((int)blockIdx.x >= Opad) {
    const int f = ((int)blockIdx.x - Opad) * 256 + (int)threadIdx.x;
    if (tables != nullptr && f < ngroups * kGroup) {
      float* dst = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(tables) +
                                            (size_t)(f / kGroup) * tbl_group_bytes(L) + (f % kGroup) * 64 * L);
      if (f < I) {
        kan_table_feature(grid + (size_t)f * L, L, dst);
      } else {  // missing feature: +inf knots (every basis zero) and zero coefficients
        for (int k = 0; k < kMaxKnots; ++k) dst[k] = __builtin_inff();
        for (int k = kMaxKnots; k < 16 * L; ++k) dst[k] = 0.0f;
      }
    }
    return;
  }
  const int o = blockIdx.x;
  const bool live = o < O;
  float mx = 0.0f;
  if (live) {
    for (int i = threadIdx.x; i < I; i += 256) {
      mx = fmaxf(mx, fabsf(wb[(size_t)o * I + i]));
      const float s = sc[(size_t)o * I + i];
      for (int c = 0; c < C; ++c) mx = fmaxf(mx, fabsf(ws[((size_t)o * I + i) * C + c] * s));
    }
  }
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (mx > 0.0f && mx < __builtin_inff()) e = 14 - ilogbf(mx);
  e = e > 100 ? 100 : (e < -100 ? -100 : e);
  const float scale = ldexpf(1.0f, e);
  if (threadIdx.x == 0) colscale[o] = ldexpf(1.0f, -e);

  const int per_group = 1 + Cp;
  const int total8 = ngroups * per_group * (kChunk / 8);  // 8 consecutive slots per item
  const int feats_per_chunk = kChunk / Cp;
  for (int idx = threadIdx.x; idx < total8; idx += 256) {
    const int q = idx / (kChunk / 8), s0 = (idx % (kChunk / 8)) * 8;
    const int g = q / per_group, sub = q % per_group;
    f16x8 h8, l8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int s = s0 + e;
      float v = 0.0f;
      if (live) {
        if (sub == 0) {
          const int f = g * kGroup + s;
          if (f < I) v = wb[(size_t)o * I + f];
        } else {
          const int f = g * kGroup + (sub - 1) * feats_per_chunk + s / Cp;
          const int c = s % Cp;
          if (f < I && c < C) v = ws[((size_t)o * I + f) * C + c] * sc[(size_t)o * I + f];
        }
      }
      v *= scale;
      const _Float16 h = (_Float16)v;
      h8[e] = h;
      l8[e] = (_Float16)(v - (float)h);
    }
    const size_t dst = ((size_t)q * Opad + o) * kChunk + s0;
    *reinterpret_cast<f16x8*>(bhi + dst) = h8;
    *reinterpret_cast<f16x8*>(blo + dst) = l8;
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
// rows are read before Q1, whose MFMAs cover that latency; the interval count is
// interleaved with Q2's MFMAs and then issues the coefficient reads, which Q3 covers; the
// cubic evaluation, split and placement are interleaved with Q4's MFMAs.  The loop body is
// one whole feature group unrolled (every chunk kind and wait count is a constant) and
// weight and table copies past the end zero-fill through the buffer descriptors, so no
// branch surrounds the MFMAs (which would make the compiler copy the accumulators).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ int swizzle64(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4);
}

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Copy chunk q's hi and lo tiles (rows n0..n0+BN-1 of [q][Opad][32]) into an LDS stage.
// A direct-to-LDS instruction writes 64 consecutive 16-byte slots (16 rows of 64 bytes);
// lane i fetches the chunk the swizzle places in slot i.  Each wave copies
// kGroupsPerWave groups of each half.
__device__ __forceinline__ void dma_chunk(__amdgpu_buffer_rsrc_t rhi, __amdgpu_buffer_rsrc_t rlo,
                                          uint8_t* stage, int q, int Opad, int n0, int wave,
                                          int lane) {
  const int r16 = lane / 4, logical = (lane % 4) ^ ((r16 >> 2) & 3);
  static_assert(kGroupsPerWave * kWaves * 16 == BN, "tile rows split evenly over waves");
#pragma unroll
  for (int i = 0; i < kGroupsPerWave; ++i) {
    const int group = wave * kGroupsPerWave + i;
    const int row = group * 16 + r16;
    const unsigned off = (unsigned)(((size_t)q * Opad + n0 + row) * 64 + 16 * logical);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rhi, (__attribute__((address_space(3))) void*)(stage + group * 1024), 16, off, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rlo, (__attribute__((address_space(3))) void*)(stage + kTileBytes + group * 1024), 16, off,
        0, 0, 0);
  }
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

// V (four fp16 values, low first) placed at fp16 slot p of an 8-slot window: slots p..p+3
// of the window get V[0..3]; values outside the window are dropped.
__device__ __forceinline__ i32x4 place4(unsigned long long V, int p) {
  const int sh = 16 * p;
  const unsigned long long left = V << (sh & 63), right = V >> ((-sh) & 63);
  const unsigned long long carry = V >> ((64 - sh) & 63), left2 = V << ((sh - 64) & 63);
  const unsigned long long lo = (sh >= 0 && sh < 64) ? left : ((sh < 0 && sh > -64) ? right : 0ull);
  const unsigned long long hi = (sh > 0 && sh < 64) ? carry : ((sh >= 64 && sh < 128) ? left2 : 0ull);
  return i32x4{(int)(unsigned)lo, (int)(unsigned)(lo >> 32), (int)(unsigned)hi, (int)(unsigned)(hi >> 32)};
}

struct TabFetch {
  f32x4 c[4];
  float tj;
  int j;
  bool inside;
};

__device__ __forceinline__ void tab_knots(const float* fe, f32x4 (&kn)[4]) {
  const f32x4* k4 = reinterpret_cast<const f32x4*>(fe);
#pragma unroll
  for (int q = 0; q < 4; ++q) kn[q] = k4[q];
}

__device__ __forceinline__ TabFetch tab_locate(float x, const f32x4 (&kn)[4], const float* fe, int L) {
  int cnt = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) cnt += (x >= kn[q].x) + (x >= kn[q].y) + (x >= kn[q].z) + (x >= kn[q].w);
  TabFetch r;
  r.j = min(max(cnt - 1, 0), L - 2);
  r.inside = cnt >= 1 && cnt <= L - 1;
  r.tj = fe[r.j];
  const f32x4* cf = reinterpret_cast<const f32x4*>(fe + kMaxKnots + 16 * r.j);
#pragma unroll
  for (int q = 0; q < 4; ++q) r.c[q] = cf[q];
  return r;
}

__device__ __forceinline__ void tab_finish(float x, const TabFetch& t, int b0, f16x8& hi, f16x8& lo) {
  const float u = x - t.tj;
  float N[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const f32x4 c = t.c[r];
    N[r] = t.inside ? fmaf(fmaf(fmaf(c.w, u, c.z), u, c.y), u, c.x) : 0.0f;
  }
  asm volatile("" : "+v"(N[0]), "+v"(N[1]), "+v"(N[2]), "+v"(N[3]));
  const f16x2 h01 = __builtin_convertvector(f32x2{N[0], N[1]}, f16x2);
  const f16x2 h23 = __builtin_convertvector(f32x2{N[2], N[3]}, f16x2);
  const f16x2 l01 = __builtin_convertvector(f32x2{N[0] - (float)h01.x, N[1] - (float)h01.y}, f16x2);
  const f16x2 l23 = __builtin_convertvector(f32x2{N[2] - (float)h23.x, N[3] - (float)h23.y}, f16x2);
  const unsigned long long H = (unsigned long long)__builtin_bit_cast(unsigned, h01) |
                               ((unsigned long long)__builtin_bit_cast(unsigned, h23) << 32);
  const unsigned long long Lw = (unsigned long long)__builtin_bit_cast(unsigned, l01) |
                                ((unsigned long long)__builtin_bit_cast(unsigned, l23) << 32);
  const int p = t.j - kOrder - b0;
  hi = __builtin_bit_cast(f16x8, place4(H, p));
  lo = __builtin_bit_cast(f16x8, place4(Lw, p));
}

template <int kCp, bool kVec4>
__global__ __launch_bounds__(kThreads) void kan_gemm(
    const float* __restrict__ x, const float* __restrict__ tables, int B, int I, int O, int L,
    int ngroups, int Opad, const _Float16* __restrict__ bhi, const _Float16* __restrict__ blo,
    const float* __restrict__ colscale, float* __restrict__ out) {
  constexpr int kStages = 4;
  constexpr int kQ = 1 + kCp;                        // chunks per feature group
  constexpr int kFeatsPerChunk = kChunk / kCp;
  constexpr int kPerStep = 2 * kGroupsPerWave;        // weight copy instructions per wave per chunk
  constexpr int kX = 8 + kCp;                         // x values per lane and row block per group
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* tbl = smem + kStages * kStageBytes;
  const int tm = (B + BM - 1) / BM, tn = Opad / BN;
  int mt, nt;
  tile_of(blockIdx.x, tm, tn, mt, nt);
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

  // x values this lane needs per group and row block: slots 0..7 the silu chunk's
  // features 8*fg..+7, slot 8+t the spline chunk t's feature.
  auto xfeat = [&](int slot) {
    return slot < 8 ? 8 * fg + slot : (slot - 8) * kFeatsPerChunk + (8 * fg) / kCp;
  };
  float xcur[2][kX], xnext[2][kX];
  auto prefetch = [&](int g) {  // past I or B: reads as 0 (against zero weights)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int row = row0 + rb * 16 + fr;
#pragma unroll
      for (int t = 0; t < kX; ++t) {
        const int f = g * kGroup + xfeat(t);
        const unsigned off = (row < B && f < I) ? (unsigned)((row * I + f) * 4) : kOutOfRange;
        xnext[rb][t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, off, 0, 0));
      }
    }
  };
  auto dma = [&](int q) { dma_chunk(rhi, rlo, smem + (q % kStages) * kStageBytes, q, Opad, n0, wave, lane); };
  auto dma_table = [&](int g) {
    for (int i = 0; i < tper; ++i) {
      const int blk = wave * tper + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rt, (__attribute__((address_space(3))) void*)(tbl + blk * 1024), 16,
          (unsigned)(g * tgb + blk * 1024 + lane * 16), 0, 0, 0);
    }
  };
  auto silu_chunk = [&](const float (&xs)[2][kX], f16x8 (&hi)[2], f16x8 (&lo)[2]) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      float v[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) v[t] = silu(xs[rb][t]);
      split8(v, hi[rb], lo[rb]);
    }
  };

  // Prologue: group 0's table, weight chunks 0..2, group 0's x, its silu activations.
  dma_table(0);
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) dma(s);
  prefetch(0);
  f16x8 ahi[2], alo[2];
  {
    float x0[2][kX];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int t = 0; t < kX; ++t) x0[rb][t] = xnext[rb][t];
    silu_chunk(x0, ahi, alo);
  }

  constexpr int kXLoads = 2 * kX;
  // vmcnt counts to 63; a smaller allowance only waits for more of the later loads.
  constexpr int kW0 = kPerStep + kXLoads > 63 ? 63 : kPerStep + kXLoads;
  constexpr int kW12 = 2 * kPerStep + kXLoads > 63 ? 63 : 2 * kPerStep + kXLoads;
  for (int g = 0; g < ngroups; ++g) {
    __syncthreads();
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
      __syncthreads();
      if (k == kQ - 1) dma_table(g + 1);
      dma(q + kStages - 1);

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
      // block is [o][b] (lane: batch row fr, registers: 4 consecutive columns).
      auto mfma_w = [&](int j0, const f16x8 (&w)[4][2]) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            acc[rb][j0 + u] = mfma16(w[u][0], ahi[rb], acc[rb][j0 + u]);
            acc[rb][j0 + u] = mfma16(w[u][1], ahi[rb], acc[rb][j0 + u]);
            acc[rb][j0 + u] = mfma16(w[u][0], alo[rb], acc[rb][j0 + u]);
          }
      };
      // The next chunk: this group's spline chunk k+1, or the next group's silu chunk.
      const bool spline_next = k + 1 < kQ;
      const int fl = spline_next ? k * kFeatsPerChunk + (8 * fg) / kCp : 0;  // feature in group
      const float* fe = reinterpret_cast<const float*>(tbl + fl * 64 * L);
      const int xs = spline_next ? 8 + k : 0;
      f16x8 nhi[2], nlo[2];
      f32x4 kn[4];
      TabFetch tf[2];
      load_w(0, wa);
      if (spline_next) tab_knots(fe, kn);
      __builtin_amdgcn_sched_barrier(0);
      mfma_w(0, wa);  // Q1
      load_w(4, wb);
      __builtin_amdgcn_sched_barrier(0);
      if (spline_next) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) tf[rb] = tab_locate(xcur[rb][xs], kn, fe, L);
      }
      mfma_w(4, wb);  // Q2, interleaved with the interval count
      load_w(8, wa);
#pragma unroll
      for (int u = 0; u < 24; ++u) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // 2 VALU
      }
      __builtin_amdgcn_sched_barrier(0);
      mfma_w(8, wa);  // Q3 covers the coefficient reads
      load_w(12, wb);
      __builtin_amdgcn_sched_barrier(0);
      if (spline_next) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) tab_finish(xcur[rb][xs], tf[rb], (8 * fg) % kCp, nhi[rb], nlo[rb]);
      } else {
        silu_chunk(xnext, nhi, nlo);
      }
      mfma_w(12, wb);  // Q4, interleaved with the evaluation
#pragma unroll
      for (int u = 0; u < 24; ++u) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // 4 VALU
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
      if constexpr (kVec4) {
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

}  // namespace kan
}  // namespace taskops
