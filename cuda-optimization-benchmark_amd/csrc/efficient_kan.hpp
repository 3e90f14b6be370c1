// efficient_kan kernels for gfx950 (instantiated by efficient_kan.hip).
//
// Op: tasks/efficient_kan/reference.py:33-51 (fp64 oracle :54-57):
//   out[b,o] = sum_i silu(x[b,i]) Wb[o,i] + sum_i sum_c B_c(x[b,i]) Ws[o,i,c] sc[o,i]
// with B_c the order-p B-spline bases on feature i's knot row (Cox-de Boor).
//
// One contraction over K = I * (1 + C') (C' = C rounded up to 8 or 16) with a three-term
// split for fp32-level accuracy: every operand v is carried as hi = fp16(v) and
// lo = fp16(v - hi), and each product as hi*hi + lo*hi + hi*lo (the dropped lo*lo term is
// ~2^-22 relative), accumulated in fp32.  The activations are the MFMAs' A operand and the
// weights the B operand.
//
// K order (spline_k): features in groups of 32; each group is one silu chunk (32 features,
// k = feature), contracted with the dense v_mfma_f32_16x16x32_f16, then C'/2 spline steps
// of 64 k.  A feature has at most four nonzero bases (the window j-3 .. j of x's knot
// interval j), and its bases are ordered so that every group of 4 k holds at most two of
// them, so the spline activations are 2:4-sparse and each step is one
// v_smfmac_f32_16x16x64_f16 per product term: a lane stores the 8 nonzero-or-paired values
// of its 16 k with 2-bit positions, and its rows' bases come from the knot row (cardinal
// cubic pieces on uniform rows, else per-interval cubics from a table).
//
// Per call, two launches: kan_pack finds each output column's power-of-two scale (so
// neither fp16 half under- or overflows), writes the weights ([Wb | Ws*sc]) in that K order
// as scaled fp16 hi/lo, [chunk of 32 k][column][32] so each chunk's tile is contiguous, and
// tabulates every feature's knot row and per-interval basis cubics; kan_fused is the
// warp-specialized GEMM (producer waves expand the activations into LDS, consumer waves
// load their weight fragments straight into registers and run the MFMAs) and undoes the
// column scale in its epilogue.
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
typedef int i32x2 __attribute__((ext_vector_type(2)));

constexpr int kGroup = 32;        // features per group
constexpr int kChunk = 32;        // k per MFMA chunk
constexpr int kMaxKnots = 16;     // fast path: grid_size + 2*order + 1 <= 16
constexpr int kOrder = 3;         // the fast path's spline order
constexpr int kRawBufferFlags = 0x00020000;
constexpr unsigned kOutOfRange = 0x80000000u;
constexpr int kStoreSystem = 17;  // buffer store cache policy sc0 | sc1: system scope, through the L2

// kan_fused tiling: a 128 x 256 output tile per workgroup of 8 waves.  Waves 0-3 are
// consumers: wave w owns all 128 batch rows (8 row blocks of 16) x output columns
// 64w .. 64w+63 (4 column blocks), 128 fp32 accumulators; it loads its weight fragments,
// reads the activations from LDS and issues the MFMAs.  Waves 4-7 are producers: producer
// p expands the activations of batch rows 32p .. 32p+31 (2 row blocks).  One producer and
// one consumer share each SIMD.
constexpr int kThreads = 512;
constexpr int kConsumerWaves = 4;
constexpr int BM = 128;
constexpr int BN = 256;
constexpr int kRB = BM / 16;                        // row blocks per tile (consumer)
constexpr int kCB = BN / 16 / kConsumerWaves;       // column blocks per consumer wave
constexpr int kActFragBytes = kRB * 2 * 64 * 16;    // hi + lo activation fragments: 16 KiB
constexpr int kActIdxBytes = kRB * 64 * 4;          // sparse positions, a pair of row blocks per 8 bytes: 2 KiB
constexpr int kActBytes = kActFragBytes + kActIdxBytes;
constexpr int kActStages = 2;
constexpr int kActAt = 0;
constexpr int kTblAt = kActAt + kActStages * kActBytes;
constexpr int kTblSetSlots = 8;                     // features per table set (C' = 8; C' = 16 uses 4)
constexpr int kTblBytes = 2 * kTblSetSlots * 64 * kMaxKnots;  // two sets of 1 KiB entries: 16 KiB
constexpr int kLdsBytes = kTblAt + kTblBytes;       // 52 KiB
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

// Whether a knot row is uniform to within rel: h > 0 and every knot within rel * h of
// t_0 + k h.  Within 1e-3 h the GEMM's direct interval lookup is exact enough.  Within
// 5e-7 h the bases are the cardinal cubic pieces to about 1e-6 of a basis value (twice the
// knot deviation, plus the fp32 evaluation), so the GEMM may evaluate those instead of the
// table's per-interval cubics: the grids efficient-kan builds, arange * h + a in fp32, are
// uniform to a few ulps (2.2e-7 h at grid_size 5, exact at 8; up to 9.5e-7 h for other
// sizes up to 13, whose rows then take the table).  The threshold bounds what the
// approximation can cost: with the reference's weight distributions (Ws 0.05 N, scaler
// 1 + 0.1 N) at I = O = 1024, knots jittered by 1e-6 h measured (CPU model of the
// evaluation) a worst output error of 0.37 of the task's atol = rtol = 1e-5 bound, and by
// 9e-6 h 3.4 times the bound, so rows that far from uniform must use the table.
// The row is passed in registers (kn[k] for k < L) and the loops are unrolled with the
// bound as a predicate, so the check is one pass of arithmetic; walking the row in memory
// with an early exit made it a chain of dependent cache round trips.
__host__ __device__ inline bool kan_knots_uniform(const float (&kn)[kMaxKnots], int L, double rel) {
  if (L < 2) return false;
  const double t0 = (double)kn[0];
  double tl = t0;
#pragma unroll
  for (int k = 1; k < kMaxKnots; ++k)
    if (k == L - 1) tl = (double)kn[k];
  const double h = (tl - t0) / (L - 1);
  if (!(h > 0.0) || !(h < 1e300)) return false;
  bool ok = true;
#pragma unroll
  for (int k = 0; k < kMaxKnots; ++k)
    if (k < L) ok = ok && __builtin_fabs((double)kn[k] - (t0 + k * h)) <= rel * h;
  return ok;
}
constexpr double kUniformRel = 1e-3;   // direct interval lookup
constexpr double kCardinalRel = 5e-7;  // cardinal pieces in place of the table's cubics

// Spacing h of a knot row as the uniformity check defines it: (t_{L-1} - t_0) / (L - 1).
__host__ __device__ inline double kan_row_spacing(const float (&kn)[kMaxKnots], int L) {
  double tl = (double)kn[0];
#pragma unroll
  for (int k = 1; k < kMaxKnots; ++k)
    if (k == L - 1) tl = (double)kn[k];
  return (tl - (double)kn[0]) / (L - 1);
}

// Interval j's cubics for a knot row uniform to 5e-7 h (kan_knots_uniform with
// kCardinalRel): on a uniform row every basis N_{k,3} with 0 <= k <= L - 5 is the cardinal
// cubic B-spline, and on interval j basis j - 3 + r is its piece 3 - r, in t = u / h:
//   piece 0  t^3 / 6                      piece 1  (1 + 3t + 3t^2 - 3t^3) / 6
//   piece 2  (4 - 6t^2 + 3t^3) / 6        piece 3  (1 - t)^3 / 6
// so the coefficient of u^c is the piece's coefficient of t^c times h^-c.  Against the fp64
// recursion on the row's own knots (kan_table_entry) it differs by the row's deviation from
// uniform, about 1e-6 of a basis value at most, the same approximation kan_fused makes when
// it evaluates these pieces itself; it needs one division where the recursion needs 32.
// ent: the interval's 16 floats.
__device__ __forceinline__ void kan_cardinal_entry(int L, int j, double h, float* ent) {
  constexpr double kPiece[4][4] = {{0.0, 0.0, 0.0, 1.0 / 6.0},
                                   {1.0 / 6.0, 0.5, 0.5, -0.5},
                                   {2.0 / 3.0, 0.0, -1.0, 0.5},
                                   {1.0 / 6.0, -0.5, 0.5, -1.0 / 6.0}};
  const double ih = 1.0 / h;
  const double ihp[4] = {1.0, ih, ih * ih, ih * ih * ih};
#pragma unroll
  for (int r = 0; r <= kOrder; ++r) {  // basis j - 3 + r; (j - 3 + r) % 4 == (j + 1 + r) % 4
    const int kb = j - kOrder + r;
    const bool exists = kb >= 0 && kb <= L - 2 - kOrder;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      ent[4 * tbl_chunk(j, (j + 1 + r) & 3) + c] = exists ? (float)(kPiece[kOrder - r][c] * ihp[c]) : 0.0f;
  }
}

// Entry j of a feature's table (ent: the entry's 16 floats): j = -1 the knot row, j in
// [0, L-1) interval j's cubics.
__device__ __forceinline__ void kan_table_entry(const float* __restrict__ knots_row, int L, int j, float* ent) {
  if (j < 0) {
    for (int k = 0; k < kMaxKnots; ++k) ent[k] = k < L ? knots_row[k] : __builtin_inff();
    return;
  }
  // The recursion for interval j only reads knots j-3 .. j+4; w[i] = t_{j-3+i} (0 outside the
  // row, never read: the index ranges below keep k >= 0 and k + p + 1 <= L - 1).  With the
  // loops unrolled every index into w, P and Q is a constant, so they stay in registers;
  // indexing a whole knot row by the thread's j instead turned each access into a chain of
  // selects over the row, and the table took 7-11 us of kan_pack's critical path.
  double w[2 * (kOrder + 1)];
#pragma unroll
  for (int i = 0; i < 2 * (kOrder + 1); ++i) {
    const int k = j - kOrder + i;
    w[i] = (k >= 0 && k < L) ? (double)knots_row[k] : 0.0;
  }
  double P[kOrder + 1][4];  // P[r]: N_{j-3+r, p} as a cubic in u
#pragma unroll
  for (int r = 0; r <= kOrder; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) P[r][c] = 0.0;
  if (w[kOrder + 1] > w[kOrder]) P[kOrder][0] = 1.0;  // N_{j,0} on [t_j, t_{j+1})
#pragma unroll
  for (int p = 1; p <= kOrder; ++p) {
    double Q[kOrder + 1][4];
#pragma unroll
    for (int r = 0; r <= kOrder; ++r) {
#pragma unroll
      for (int c = 0; c < 4; ++c) Q[r][c] = 0.0;
      const int k = j - kOrder + r;  // t_k = w[r], t_j = w[kOrder]
      if (r < kOrder - p || k < 0 || k > L - 2 - p) continue;
      const double d1 = w[r + p] - w[r], d2 = w[r + p + 1] - w[r + 1];
      if (d1 != 0.0) {  // (u + (t_j - t_k)) / d1 * N_{k,p-1}
        const double a = (w[kOrder] - w[r]) / d1, b = 1.0 / d1;
#pragma unroll
        for (int c = 3; c >= 0; --c) Q[r][c] += a * P[r][c] + (c > 0 ? b * P[r][c - 1] : 0.0);
      }
      if (d2 != 0.0 && r < kOrder) {  // ((t_{k+p+1} - t_j) - u) / d2 * N_{k+1,p-1}
        const double a = (w[r + p + 1] - w[kOrder]) / d2, b = -1.0 / d2;
#pragma unroll
        for (int c = 3; c >= 0; --c) Q[r][c] += a * P[r + 1][c] + (c > 0 ? b * P[r + 1][c - 1] : 0.0);
      }
    }
#pragma unroll
    for (int r = 0; r <= kOrder; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) P[r][c] = Q[r][c];
  }
#pragma unroll
  for (int r = 0; r <= kOrder; ++r)  // basis j - 3 + r; (j - 3 + r) % 4 == (j + 1 + r) % 4
#pragma unroll
    for (int c = 0; c < 4; ++c) ent[4 * tbl_chunk(j, (j + 1 + r) & 3) + c] = (float)P[r][c];
}


// ---------------------------------------------------------------------------------------
// Weight preparation, one launch (kan_pack): each output column's scale, the GEMM's weight
// operand, and the basis tables.
// bhi/blo: [nchunks][Opad][32] fp16; chunk q = g*(1+Cp) + sub; sub 0 holds Wb[o, 32g + s],
// subs 1 .. Cp hold (Ws*sc)[o, f, c] at the place spline_k gives feature f % 32 of group g
// and the basis order spline_basis (zero past I, O or C), all times 2^e.  colscale[o] =
// 2^-e with e chosen so max|column| * 2^e is in [2^14, 2^15), so neither fp16 half under-
// or overflows.
// ---------------------------------------------------------------------------------------
// The GEMM's K order within a feature group (32 features): chunk 0 holds silu(x) of the 32
// features (k = feature); chunks 1 .. C' hold the spline bases, in C'/2 steps of 64 k (two
// chunks each) that the sparse MFMA consumes whole.  In step u, lane quarter q of the MFMA
// supplies k = 16 q .. 16 q + 15 of the step:
//   C' = 8:  features 8q + 2u and 8q + 2u + 1, 8 slots each, bases in the order 0 2 4 6 1 3 5 7;
//   C' = 16: feature 8q + u, 16 slots, bases in the order 0 4 8 12 1 5 9 13 2 6 10 14 3 7 11 15.
// Each group of 4 slots then holds at most two of a feature's four nonzero bases (the
// window j-3 .. j has two even and two odd bases, and one basis per residue mod 4), the
// 2:4 pattern of v_smfmac_f32_16x16x64_f16.  Over a group a lane quarter's features are the
// contiguous run 8q .. 8q + 7.
template <int kCp>
__host__ __device__ inline void spline_k(int fl, int& sub, int& slot) {
  const int q = fl / 8;
  const int u = kCp == 8 ? (fl % 8) / 2 : fl % 8;
  const int k = kCp == 8 ? 16 * q + 8 * (fl % 2) : 16 * q;  // first k of the feature's slots in its step
  sub = 1 + 2 * u + k / 32;
  slot = k % 32;
}
// Basis in slot s of a feature's C' slots.
template <int kCp>
__host__ __device__ constexpr int spline_basis(int s) {
  return kCp == 8 ? (s < 4 ? 2 * s : 2 * (s - 4) + 1) : 4 * (s % 4) + s / 4;
}

// Basis table entries first .. first + kPackThreads - 1 (L per feature: the knot row and
// the L - 1 intervals, 64 bytes each), one per thread.  Each thread builds its entry in LDS;
// then every thread stores 16-byte chunks of consecutive entries, so a wave's store covers
// 1 KiB of the table (entries are consecutive in memory within a feature group).  Written
// one float at a time from the thread that computed it, each store instruction touched 64
// separate lines and the 24 table workgroups at BASELINE took about 6 us.  Returns this
// thread's flags: bit 0 every knot row it wrote is uniform to 1e-3 h, bit 1 to 5e-7 h
// (kan_knots_uniform); the caller combines them.
constexpr int kTableThreads = 512;
__device__ __forceinline__ int kan_tables_range(int first, const float* __restrict__ grid, int I, int L,
                                                int ngroups, float* __restrict__ tables) {
  __shared__ f32x4 stage[kTableThreads * 4];  // entry e at stage[4e .. 4e + 3]
  bool uniform = true, cardinal = true;
  const int tid = (int)threadIdx.x;
  const int nent = ngroups * kGroup * L;  // entries past it belong to no group
  {
    const int idx = first + tid;
    const int f = idx / L, j = idx % L - 1;
    float* ent = reinterpret_cast<float*>(stage + 4 * tid);
    if (idx < nent && f < I) {
      float kn[kMaxKnots];
#pragma unroll
      for (int k = 0; k < kMaxKnots; ++k) kn[k] = k < L ? grid[(size_t)f * L + k] : 0.0f;
      const bool row_cardinal = kan_knots_uniform(kn, L, kCardinalRel);
      if (j >= 0 && row_cardinal)
        kan_cardinal_entry(L, j, kan_row_spacing(kn, L), ent);
      else
        kan_table_entry(grid + (size_t)f * L, L, j, ent);
      if (j < 0) {
        uniform = uniform && kan_knots_uniform(kn, L, kUniformRel);
        cardinal = cardinal && row_cardinal;
      }
    } else if (idx < nent) {  // missing feature: knots 0, 1, 2, ... and zero coefficients
      for (int k = 0; k < 16; ++k) ent[k] = j < 0 ? (float)k : 0.0f;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + kTableThreads * i;  // chunk c % 4 of entry c / 4
    const int idx = first + c / 4;
    if (idx < nent) {
      const int f = idx / L, e = idx % L;
      uint8_t* dst = reinterpret_cast<uint8_t*>(tables) + (size_t)(f / kGroup) * tbl_group_bytes(L) +
                     ((f % kGroup) * L + e) * 64 + 16 * (c % 4);
      *reinterpret_cast<f32x4*>(dst) = stage[c];
    }
  }
  return (uniform ? 1 : 0) | (cardinal ? 2 : 0);
}

// kan_pack: the first tblocks workgroups build the basis tables, kPackThreads entries each
// (kan_tables_range), and write one knot-row flag word each; they need nothing from the
// packing, so they run beside it.  Workgroup tblocks + t owns the column pair 2t, 2t + 1
// (pack_columns) with all 8 waves: lanes 0-31 of a wave take column 2t and lanes 32-63
// column 2t + 1, lane fl of a half feature fl of a group (32 features).  Each wave takes
// pack_runs runs of a batch (4 for Cp = 8, 1 for Cp = 16): wave w takes groups w, w + 8,
// w + 16, ... of the batch, so a run's loads cover 1 KiB (Cp = 8) of one column's
// contiguous Ws rows per half-wave.  Pass 1 reduces each column's max |w| over Wb, sc and Ws to
// colscale[o] (the waves combine through LDS); pass 2 writes the hi/lo weights: lane
// (column o, feature f) writes all of f's bases, one run of Cp slots at spline_k(f % 32) in
// the permuted basis order, and lanes with f % 32 < 4 also write silu slots 8 (f % 32) .. +7.
// The pair's two 64-byte halves of a chunk make one 128-byte line and both come from one
// store instruction, so every store writes whole lines.  With one column per wave (each
// line's halves written by two waves) the same data movement took 23.5 us against 18.4 us
// (a `_work` probe of this phase alone).  When one batch covers every feature (I <= 1024 for
// Cp = 8, I <= 256 for Cp = 16) it stays in registers between the passes; wider inputs read
// each run again in pass 2 (from the L2 or the Infinity Cache).  Workgroup tblocks also
// zeroes kan_fused's split-K arrival counters (their place in the workspace moves with the
// shape, so every call starts them from zero).
// At BASELINE the columns are 512 workgroups, as many as are resident at once, and the 24
// table workgroups hold slots until they finish, so table time delays the last column
// workgroups.  Measured (one box, median of 150): 15.6 us without tables, 21.7 us with
// the recursion indexing whole knot rows, 18.8 us with its 8-knot window, 18.7 us with the
// closed form for cardinal rows as well; building the tables inside the column workgroups,
// before or after their columns, measured 23.7-26.7 us.
constexpr int kPackCols = 2;
constexpr int kPackWaves = 8;
constexpr int kPackThreads = kPackWaves * kWave;
// Runs per wave and batch (a batch is kPackWaves * runs groups): 4 for Cp = 8 and 1 for
// Cp = 16, which keeps a batch's rows within the 128 registers of four waves per SIMD.
// With 2 runs for Cp = 16 the reference's timed shape (I = 256, one group per wave) took
// 78.0-78.2 us per call against 74.6-75.9 us with 1 run (A/B on one box, both orders).
template <int kCp>
constexpr int pack_runs() { return kCp == 8 ? 4 : 1; }
static_assert(kPackThreads == kTableThreads, "a table workgroup is one kan_pack workgroup");
static_assert(kPackCols * kGroup == kWave, "a wave's halves are the pair's two columns");
// Workgroup t's column pair (pass 1 and pass 2 above).
template <int kCp, bool kVecW>
__device__ __forceinline__ void pack_columns(int t, const float* __restrict__ wb, const float* __restrict__ ws,
                                             const float* __restrict__ sc, int I, int O, int C, int Opad,
                                             float* __restrict__ colscale, _Float16* __restrict__ bhi,
                                             _Float16* __restrict__ blo, int ngroups, unsigned* __restrict__ counters,
                                             int ncounters) {
  static_assert(kCp % 8 == 0, "whole 8-slot runs");
  __shared__ float colmax[kPackCols][kPackWaves];
  constexpr int kSub = 1 + kCp;
  constexpr int kPackRuns = pack_runs<kCp>();
  constexpr int kPackBatch = kPackWaves * kPackRuns;
  if (t == 0)
    for (int i = threadIdx.x; i < ncounters; i += kPackThreads) counters[i] = 0u;
  const int lane = (int)threadIdx.x % kWave, wave = (int)threadIdx.x / kWave;
  const int oc = lane / kGroup, fl = lane % kGroup;
  const int o0 = t * kPackCols, o = o0 + oc;
  const bool col = o < O;

  // Pass 1: max over each column.  max_c |ws * s| = |s| * max_c |ws| exactly (rounding is
  // monotonic).  Every load of a batch is a buffer load with no branch around it (an offset
  // past the buffer reads zero for a missing feature, column or basis), so all of them are
  // in flight before the first is used: behind per-run branches the compiler waited for
  // each run's loads before issuing the next run's, one memory round trip per run.
  // The descriptors start at the pair's first column and cover its columns below O, so
  // their 32-bit offsets need only two columns' rows to fit (Ws as a whole may pass 2 GiB);
  // a pair past O reads nothing.
  const int ncols = O - o0 >= kPackCols ? kPackCols : (O > o0 ? O - o0 : 0);
  const size_t obase = ncols > 0 ? (size_t)o0 : 0;
  const __amdgpu_buffer_rsrc_t rwb = make_rsrc(wb + obase * I, (size_t)ncols * I * 4);
  const __amdgpu_buffer_rsrc_t rsc = make_rsrc(sc + obase * I, (size_t)ncols * I * 4);
  const __amdgpu_buffer_rsrc_t rws = make_rsrc(ws + obase * I * C, (size_t)ncols * I * C * 4);
  const unsigned cwb = (unsigned)oc * (unsigned)I * 4u;               // this lane's column in rwb, rsc
  const unsigned cws = (unsigned)oc * (unsigned)I * (unsigned)C * 4u;  // and in rws
  float wbv[kPackRuns], scv[kPackRuns], rows[kPackRuns][kCp];
  // Run u of batch bt is group bt * kPackBatch + u * kPackWaves + wave; its loads go into
  // wbv[u], scv[u] and rows[u].
  auto load_run = [&](int bt, int u) {
    const int f = (bt * kPackBatch + u * kPackWaves + wave) * kGroup + fl;
    const bool ok = col && f < I;
    const unsigned off = ok ? cwb + (unsigned)f * 4u : kOutOfRange;
    wbv[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rwb, off, 0, 0));
    scv[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsc, off, 0, 0));
    const unsigned row = cws + (unsigned)f * (unsigned)C * 4u;
    if constexpr (kVecW) {  // C % 4 == 0 and ws 16-byte aligned: 16-byte row loads
#pragma unroll
      for (int c4 = 0; c4 < kCp / 4; ++c4) {
        const unsigned o4 = ok && 4 * c4 < C ? row + 16u * c4 : kOutOfRange;
        const f32x4 w4 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rws, o4, 0, 0));
#pragma unroll
        for (int e = 0; e < 4; ++e) rows[u][4 * c4 + e] = w4[e];
      }
    } else {
#pragma unroll
      for (int c = 0; c < kCp; ++c) {
        const unsigned o1 = ok && c < C ? row + 4u * c : kOutOfRange;
        rows[u][c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rws, o1, 0, 0));
      }
    }
  };
  auto load_batch = [&](int bt) {
#pragma unroll
    for (int u = 0; u < kPackRuns; ++u) load_run(bt, u);
  };
  const int nbatch = (ngroups + kPackBatch - 1) / kPackBatch;
  float mx = 0.0f;
#pragma unroll 1
  for (int bt = 0; bt < nbatch; ++bt) {
    load_batch(bt);
#pragma unroll
    for (int u = 0; u < kPackRuns; ++u) {
      float m = 0.0f;
#pragma unroll
      for (int c = 0; c < kCp; ++c) m = fmaxf(m, fabsf(rows[u][c]));
      mx = fmaxf(mx, fmaxf(fabsf(wbv[u]), fabsf(scv[u]) * m));
    }
  }
  for (int off = kGroup / 2; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));  // within a half
  if (fl == 0) colmax[oc][wave] = mx;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kPackWaves; ++w) mx = fmaxf(mx, colmax[oc][w]);
  int e = 0;
  if (mx > 0.0f && mx < __builtin_inff()) e = 14 - ilogbf(mx);
  e = e > 100 ? 100 : (e < -100 ? -100 : e);
  if (wave == 0 && fl == 0) colscale[o] = ldexpf(1.0f, -e);
  const float scale = ldexpf(1.0f, e);  // 2^e, exact

  // Pass 2: the scaled hi/lo weights of every group (zero past I and O).  The pair's two
  // columns of a chunk are one 128-byte line, and a wave writes both halves, so each store
  // instruction writes whole lines.
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
  // Feature fl's bases in the GEMM's sparse K order (spline_k): one run of C' slots, the
  // bases permuted so every group of 4 slots holds at most two of the four nonzero ones.
  auto put_spline = [&](int g, const float (&v)[kCp]) {
    int sub, slot;
    spline_k<kCp>(fl, sub, slot);
    float w[kCp];
#pragma unroll
    for (int s = 0; s < kCp; ++s) w[s] = v[spline_basis<kCp>(s)];
#pragma unroll
    for (int h = 0; h < kCp / 8; ++h) put(g, sub, slot + 8 * h, w + 8 * h);
  };
  // Lane fl < 4 of a half takes the silu weights of features 8 fl .. +7 of its group from
  // the lanes that loaded them.
  auto write_run = [&](int bt, int u) {
    const int g = bt * kPackBatch + u * kPackWaves + wave;
    float v[kCp], silu[8];
#pragma unroll
    for (int c = 0; c < kCp; ++c) v[c] = rows[u][c] * scv[u];
#pragma unroll
    for (int k = 0; k < 8; ++k) silu[k] = __shfl(wbv[u], (lane & kGroup) + ((8 * (lane & 3) + k) & (kGroup - 1)), kWave);
    if (g < ngroups) {
      put_spline(g, v);
      if (fl < 4) put(g, 0, 8 * fl, silu);
    }
  };
  if (nbatch == 1) {  // pass 1's registers hold the column pair's data
#pragma unroll
    for (int u = 0; u < kPackRuns; ++u) write_run(0, u);
    return;
  }
  // Wider inputs: each run again, loaded and written in turn (one run's registers live).
#pragma unroll 1
  for (int bt = 0; bt < nbatch; ++bt)
#pragma unroll
    for (int u = 0; u < kPackRuns; ++u) {
      load_run(bt, u);
      write_run(bt, u);
    }
}

// Four waves per SIMD (at most 128 VGPRs): two workgroups per CU, so 512 column workgroups
// are resident at once; at 132 VGPRs it was one per CU and twice as slow.
template <int kCp, bool kVecW>
__global__ __launch_bounds__(kPackThreads) __attribute__((amdgpu_waves_per_eu(4))) void kan_pack(
    const float* __restrict__ wb, const float* __restrict__ ws, const float* __restrict__ sc, int I,
    int O, int C, int Opad, float* __restrict__ colscale, _Float16* __restrict__ bhi,
    _Float16* __restrict__ blo, const float* __restrict__ grid, int L, int ngroups, int tblocks,
    float* __restrict__ tables, int* __restrict__ uflags, unsigned* __restrict__ counters,
    int ncounters) {
  const int t = (int)blockIdx.x - tblocks;
  if (t < 0) {
    const int b = (int)blockIdx.x;
    const int flags = kan_tables_range(b * kTableThreads, grid, I, L, ngroups, tables);
    const bool uniform = __syncthreads_and(flags & 1), cardinal = __syncthreads_and(flags & 2);
    if (threadIdx.x == 0) uflags[b] = (uniform ? 1 : 0) | (cardinal ? 2 : 0);
    return;
  }
  pack_columns<kCp, kVecW>(t, wb, ws, sc, I, O, C, Opad, colscale, bhi, blo, ngroups, counters, ncounters);
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

// The four cubics at u = x - t_j: N[m] is the basis of the window [j-3, j] with index = m
// (mod 4); zero outside the knot span, and the table holds zero coefficients for bases
// outside [0, C).
__device__ __forceinline__ void tab_values(float x, const TabFetch& t, float (&N)[4]) {
  const float u = x - t.tj;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const f32x4 c = t.c[m];
    N[m] = t.inside ? fmaf(fmaf(fmaf(c.w, u, c.z), u, c.y), u, c.x) : 0.0f;
  }
}

// Two bases at consecutive positions first, first + 1 of a group of 4 slots (values v0, v1)
// as a sparse pair: the positions clamped into the group (a pair past its ends holds bases
// outside [0, C'), whose values are zero) and the values that land on them.
__device__ __forceinline__ void sparse_pair(int first, float v0, float v1, float& a, float& b, unsigned& pos) {
  const int p = min(max(first, 0), 2);
  const int d = p - first;  // 1, 0, -1 or -2
  a = d == 0 ? v0 : (d == 1 ? v1 : 0.0f);
  b = d == 0 ? v1 : (d == -1 ? v0 : 0.0f);
  pos = (unsigned)p | ((unsigned)(p + 1) << 2);
}

// One feature's compressed A values for C' = 8 (4 values: group 0 the even bases, group 1
// the odd ones) and their 8 position bits.
__device__ __forceinline__ void sparse8(int j, const float (&N)[4], float* v, unsigned& bits) {
  const int e0 = (j & 1) ? j - 3 : j - 2;  // the window's first even basis
  const int o0 = (j & 1) ? j - 2 : j - 3;  // and first odd one
  // N[m] holds the basis = m (mod 4): e0 and e0 + 2 are 0 and 2 (mod 4) in some order
  const bool es = (e0 & 2) != 0, os = (o0 & 2) != 0;
  unsigned pe, po;
  sparse_pair(e0 >> 1, es ? N[2] : N[0], es ? N[0] : N[2], v[0], v[1], pe);
  sparse_pair((o0 - 1) >> 1, os ? N[3] : N[1], os ? N[1] : N[3], v[2], v[3], po);
  bits = pe | (po << 4);
}

// One feature's compressed A values for C' = 16 (8 values: group r the bases = r (mod 4),
// one of them nonzero, paired with a zero at the neighbouring position) and 16 position bits.
__device__ __forceinline__ void sparse16(int j, const float (&N)[4], float* v, unsigned& bits) {
  bits = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int b = j - 3 + ((r - (j - 3)) & 3);  // the window's basis = r (mod 4)
    const int pos = b >> 2;                     // its position in group r (-1: no such basis)
    const int p = pos < 0 ? 0 : (pos & ~1);
    const bool odd = pos >= 0 && (pos & 1);
    v[2 * r] = odd ? 0.0f : N[r];
    v[2 * r + 1] = odd ? N[r] : 0.0f;
    bits |= ((unsigned)p | ((unsigned)(p + 1) << 2)) << (4 * r);
  }
}

// The four bases j-3 .. j nonzero on interval j of a uniform knot row, at t = (x - t_j) / h in
// [0, 1): the cardinal cubic B-spline pieces (1-t)^3/6, t^3/2 - t^2 + 2/3,
// -t^3/2 + t^2/2 + t/2 + 1/6 and t^3/6.  Bases outside [0, C) and x outside the knot span
// give zero.
__device__ __forceinline__ void cardinal_pieces(float t, float (&P)[4]) {
  const float t2 = t * t, t3 = t2 * t, s = 1.0f - t;
  P[0] = s * s * s * (1.0f / 6.0f);
  P[1] = fmaf(0.5f, t3, 2.0f / 3.0f - t2);
  P[2] = fmaf(-0.5f, t3, fmaf(0.5f, t2 + t, 1.0f / 6.0f));
  P[3] = t3 * (1.0f / 6.0f);
}

__device__ __forceinline__ void mask_window(int j, int C, bool inside, float (&P)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int b = j - 3 + i;
    P[i] = (inside && b >= 0 && b < C) ? P[i] : 0.0f;
  }
}

// A window needs neither the mask nor sparse_pair's clamping when x lies inside the knot
// span and all four bases j-3 .. j exist (3 <= j <= C - 1).
__device__ __forceinline__ bool window_whole(int j, int C, bool inside) { return inside && j >= 3 && j < C; }

// sparse8w for a whole window (window_whole): the first even basis is 2 ((j - 2) >> 1) and
// the first odd one 2 ((j - 3) >> 1) + 1, both pairs inside their groups, so the positions
// need no clamping: the same values and bits as sparse8w.
__device__ __forceinline__ void sparse8w_whole(int j, const float (&P)[4], float* v, unsigned& bits) {
  const bool jo = (j & 1) != 0;
  v[0] = jo ? P[0] : P[1];
  v[1] = jo ? P[2] : P[3];
  v[2] = jo ? P[1] : P[0];
  v[3] = jo ? P[3] : P[2];
  const unsigned fe = (unsigned)((j - 2) >> 1), fo = (unsigned)((j - 3) >> 1);
  bits = (5u * fe + 4u) | ((5u * fo + 4u) << 4);  // p | (p + 1) << 2 per group
}

// sparse8 from the bases in window order (P[i] is basis j - 3 + i).
__device__ __forceinline__ void sparse8w(int j, const float (&P)[4], float* v, unsigned& bits) {
  const bool jo = (j & 1) != 0;  // the first even basis is j - 3 (j odd) or j - 2
  unsigned pe, po;
  sparse_pair(jo ? (j - 3) >> 1 : (j - 2) >> 1, jo ? P[0] : P[1], jo ? P[2] : P[3], v[0], v[1], pe);
  sparse_pair(jo ? (j - 3) >> 1 : (j - 4) >> 1, jo ? P[1] : P[0], jo ? P[3] : P[2], v[2], v[3], po);
  bits = pe | (po << 4);
}

// sparse16 from the bases in window order.
__device__ __forceinline__ void sparse16w(int j, const float (&P)[4], float* v, unsigned& bits) {
  float N[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = (r - (j - 3)) & 3;  // window index of the basis = r (mod 4)
    N[r] = i == 0 ? P[0] : (i == 1 ? P[1] : (i == 2 ? P[2] : P[3]));
  }
  sparse16(j, N, v, bits);
}

// kVec: O and I multiples of 4 and out, x 16-byte aligned (16-byte x loads); otherwise
// 4-byte ones.  kUniform: every knot row passed kan_knots_uniform.

// ---------------------------------------------------------------------------------------
// kan_fused: the warp-specialized GEMM over the 2:4-sparse spline activations.
//
// Steps: per feature group, step 0 is the silu chunk (32 k, dense v_mfma_f32_16x16x32_f16)
// and steps 1 .. C'/2 are the spline steps of 64 k (v_smfmac_f32_16x16x64_f16, the
// activations the sparse A operand: 8 stored values per lane with 2-bit positions, the
// weights the dense B operand).  The activations are the A operand of both kinds, so a
// consumer lane's accumulator holds output column n0 + 64 w + 16 cb + lane % 16 of batch
// rows m0 + 16 rb + 4 (lane / 16) + 0..3.
//
// Each product is hi*hi + lo*hi + hi*lo; a step is consumed in two phases: H (hi_a * hi_w
// and lo_a * hi_w) from the step's hi weight plane, then L (hi_a * lo_w) from its lo plane.
// A consumer wave is the only reader of its 64 weight columns, so it loads its weight
// fragments straight into registers, a phase ahead: lo(s) during phase H(s), hi(s+1) during
// phase L(s).  One barrier per step: A(s) publishes step s's activations and tells the
// producers the consumers are done with step s-1's stage (the consumers arrive before phase
// L's last pair, whose activations are in registers by then, and read step s's first pair
// during it).
//   producers, between A(s) and A(s+1): refill the table set step s's features used, load
//     the next group's x (at a group's silu step), evaluate, pack and split step s+1's
//     activations and write them to stage (s+1) % 2; wait for the table set and x.
//
// LDS (kLdsBytes): 2 activation stages of 18 KiB ([row block][hi, lo][lane] x 16 B, then
// the positions [row block pair][lane][2] x 4 B) and the basis-table window, two sets of 8 (C' = 8)
// or 4 (C' = 16) feature entries: spline step u's features in set u % 2.
// ---------------------------------------------------------------------------------------

template <int kCp, bool kVec>
struct Producer {
  static constexpr int kS = kCp / 2;                       // spline steps per group
  static constexpr int kQ = 1 + kS;                        // steps per group
  static constexpr int kX = 8;                             // x values per row block per group
  static constexpr int kSetFeat = kCp == 8 ? 8 : 4;        // features per table set
  static constexpr int kTableCopies = kSetFeat / 4;        // per producer wave per set

  uint8_t* smem;
  __amdgpu_buffer_rsrc_t rx, rt;
  int I, L, B;
  int g0, nlg;
  int lane, fr, fq, pw;
  int row[2];      // this lane's batch rows (global) for its two row blocks
  bool uniform;    // every knot row is uniform: direct interval lookup
  bool cardinal;   // every knot row is uniform to 5e-7 h: cardinal pieces, no table cubics
  int C;           // bases per feature
  int tgb;

  // The table entries of spline step u's features of group lg into set u % 2: this wave
  // copies the features of slots kTableCopies * pw ..; a feature's 64 L bytes are 4 L lanes
  // of one direct-to-LDS instruction.
  __device__ __forceinline__ void copy_table_set(int lg, int u) const {
#pragma unroll
    for (int i = 0; i < kTableCopies; ++i) {
      const int slot = kTableCopies * pw + i;
      const int fl = kCp == 8 ? 8 * (slot / 2) + 2 * u + slot % 2 : 8 * slot + u;
      if (lane < 4 * L) {
        const unsigned off = (unsigned)((size_t)(g0 + lg) * tgb + fl * 64 * L + lane * 16);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rt, (__attribute__((address_space(3))) void*)(smem + kTblAt + ((u % 2) * kSetFeat + slot) * 64 * L), 16,
            off, 0, 0, 0);
      }
    }
  }

  // x at this lane's features 8 fq .. 8 fq + 7 of group lg (past I or B: 0).
  __device__ __forceinline__ void load_x(int lg, float (&xs)[2][kX]) const {
    const int g = g0 + lg;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      if constexpr (kVec) {  // I % 4 == 0: a 4-feature run is wholly inside or past I
#pragma unroll
        for (int v = 0; v < kX / 4; ++v) {
          const int f = g * kGroup + 8 * fq + 4 * v;
          const unsigned off = (row[rb] < B && f < I) ? (unsigned)(((size_t)row[rb] * I + f) * 4) : kOutOfRange;
          const f32x4 val = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
#pragma unroll
          for (int e = 0; e < 4; ++e) xs[rb][4 * v + e] = val[e];
        }
      } else {
#pragma unroll
        for (int t = 0; t < kX; ++t) {
          const int f = g * kGroup + 8 * fq + t;
          const unsigned off = (row[rb] < B && f < I) ? (unsigned)(((size_t)row[rb] * I + f) * 4) : kOutOfRange;
          xs[rb][t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, off, 0, 0));
        }
      }
    }
  }

  // Both row blocks' basis values of one feature (its table entry at `fe`): the knots are
  // read once for the two, and the two lookups' table reads go out together.
  __device__ __forceinline__ void feature_values(const float* fe, float x0, float x1, float (&N0)[4], float (&N1)[4],
                                                 int& j0, int& j1) const {
    TabFetch t0, t1;
    if (uniform) {
      const f32x2 k01 = *reinterpret_cast<const f32x2*>(fe);
      const float inv_h = __builtin_amdgcn_rcpf(k01.y - k01.x);
      t0 = tab_locate_uniform(x0, k01.x, inv_h, fe, L);
      t1 = tab_locate_uniform(x1, k01.x, inv_h, fe, L);
    } else {
      f32x4 kn[4];
      tab_knots(fe, kn);
      t0 = tab_locate_count(x0, kn, fe, L);
      t1 = tab_locate_count(x1, kn, fe, L);
    }
    tab_values(x0, t0, N0);
    tab_values(x1, t1, N1);
    j0 = t0.j;
    j1 = t1.j;
  }

  // Both row blocks' bases of one feature on a cardinal knot row, in window order: the
  // knots t_0, t_1 read once for the two, then each row's interval knot t_j.
  __device__ __forceinline__ void cardinal_values(const float* fe, float x0, float x1, float (&P0)[4], float (&P1)[4],
                                                  int& j0, int& j1, bool& in0, bool& in1) const {
    const f32x2 k01 = *reinterpret_cast<const f32x2*>(fe);
    const float inv_h = __builtin_amdgcn_rcpf(k01.y - k01.x);
    const int r0 = (int)__builtin_floorf((x0 - k01.x) * inv_h), r1 = (int)__builtin_floorf((x1 - k01.x) * inv_h);
    j0 = min(max(r0, 0), L - 2);
    j1 = min(max(r1, 0), L - 2);
    const float tj0 = fe[j0], tj1 = fe[j1];
    in0 = r0 == j0;
    in1 = r1 == j1;
    cardinal_pieces((x0 - tj0) * inv_h, P0);
    cardinal_pieces((x1 - tj1) * inv_h, P1);
  }

  // Step j's activations of a group, both of this wave's row blocks, into stage `st`: j = 0
  // the silu chunk (slots 8 fq .. 8 fq + 7 from the lane's 8 x values), else spline step
  // u = j - 1 (the lane's features 2u, 2u + 1 of its run for C' = 8, u for C' = 16).
  // When every lane's windows are whole (x inside the knot span, all four bases in [0, C)),
  // the wave packs without masks or position clamping.
  template <int kJ>
  __device__ __forceinline__ void prepare(uint8_t* st, const float (&xs)[2][kX]) const {
    float v[2][8];
    unsigned bits[2] = {0u, 0u};
    if constexpr (kJ == 0) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int t = 0; t < 8; ++t) v[rb][t] = silu(xs[rb][t]);
      }
    } else {
      constexpr int u = kJ - 1;
      const uint8_t* set = smem + kTblAt + (u % 2) * kSetFeat * 64 * L;
      if constexpr (kCp == 8) {
        float Na[2][4], Nb[2][4];
        int ja[2], jb[2];
        if (cardinal) {
          bool ia[2], ib[2];
          cardinal_values(reinterpret_cast<const float*>(set + (2 * fq) * 64 * L), xs[0][2 * u], xs[1][2 * u], Na[0],
                          Na[1], ja[0], ja[1], ia[0], ia[1]);
          cardinal_values(reinterpret_cast<const float*>(set + (2 * fq + 1) * 64 * L), xs[0][2 * u + 1],
                          xs[1][2 * u + 1], Nb[0], Nb[1], jb[0], jb[1], ib[0], ib[1]);
          const bool whole = window_whole(ja[0], C, ia[0]) && window_whole(ja[1], C, ia[1]) &&
                             window_whole(jb[0], C, ib[0]) && window_whole(jb[1], C, ib[1]);
          if (__builtin_amdgcn_ballot_w64(!whole) == 0) {  // the whole wave: no masks, no clamping
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
              unsigned ba, bb;
              sparse8w_whole(ja[rb], Na[rb], v[rb], ba);
              sparse8w_whole(jb[rb], Nb[rb], v[rb] + 4, bb);
              bits[rb] = ba | (bb << 8);
            }
          } else {
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
              unsigned ba, bb;
              mask_window(ja[rb], C, ia[rb], Na[rb]);
              mask_window(jb[rb], C, ib[rb], Nb[rb]);
              sparse8w(ja[rb], Na[rb], v[rb], ba);
              sparse8w(jb[rb], Nb[rb], v[rb] + 4, bb);
              bits[rb] = ba | (bb << 8);
            }
          }
        } else {
        feature_values(reinterpret_cast<const float*>(set + (2 * fq) * 64 * L), xs[0][2 * u], xs[1][2 * u], Na[0],
                       Na[1], ja[0], ja[1]);
        feature_values(reinterpret_cast<const float*>(set + (2 * fq + 1) * 64 * L), xs[0][2 * u + 1],
                       xs[1][2 * u + 1], Nb[0], Nb[1], jb[0], jb[1]);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          unsigned ba, bb;
          sparse8(ja[rb], Na[rb], v[rb], ba);
          sparse8(jb[rb], Nb[rb], v[rb] + 4, bb);
          bits[rb] = ba | (bb << 8);
        }
        }
      } else {
        float N[2][4];
        int jj[2];
        if (cardinal) {
          bool in[2];
          cardinal_values(reinterpret_cast<const float*>(set + fq * 64 * L), xs[0][u], xs[1][u], N[0], N[1], jj[0],
                          jj[1], in[0], in[1]);
          const bool whole = window_whole(jj[0], C, in[0]) && window_whole(jj[1], C, in[1]);
          if (__builtin_amdgcn_ballot_w64(!whole) != 0) {  // some lane's window needs the mask
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) mask_window(jj[rb], C, in[rb], N[rb]);
          }
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) sparse16w(jj[rb], N[rb], v[rb], bits[rb]);
        } else {
          feature_values(reinterpret_cast<const float*>(set + fq * 64 * L), xs[0][u], xs[1][u], N[0], N[1], jj[0],
                         jj[1]);
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) sparse16(jj[rb], N[rb], v[rb], bits[rb]);
        }
      }
    }
    f16x8 hi[2], lo[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) split8(v[rb], hi[rb], lo[rb]);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int frag = 2 * pw + rb;
      *reinterpret_cast<f16x8*>(st + ((frag * 2 + 0) * 64 + lane) * 16) = hi[rb];
      *reinterpret_cast<f16x8*>(st + ((frag * 2 + 1) * 64 + lane) * 16) = lo[rb];
    }
    // Both row blocks' positions side by side: the consumers read a pair's in one 8-byte read.
    if constexpr (kJ > 0)
      *reinterpret_cast<i32x2*>(st + kActFragBytes + (pw * 64 + lane) * 8) = i32x2{(int)bits[0], (int)bits[1]};
  }

  // Step s = lg * kQ + kJ (the consumers' phases of step s run meanwhile): see the
  // schedule above.  kLast: lg is the workgroup's last group.
  template <bool kLast, int kJ>
  __device__ __forceinline__ void step(int lg, float (&xcur)[2][kX], float (&xnext)[2][kX]) const {
    const int s = lg * kQ + kJ;
    constexpr bool kNext = !kLast || kJ + 1 < kQ;        // step s + 1 exists
    constexpr int kNJ = (kJ + 1) % kQ;                   // its position in its group
    // The table set step s (spline step kJ - 1) used is refilled for spline step kJ + 1,
    // of this group or the next.
    constexpr int kU2 = kJ + 1;
    constexpr bool kRefill = kJ >= 1 && (kU2 < kS || !kLast);
    constexpr bool kXNext = kJ == 0 && !kLast;
    uint8_t* st = smem + kActAt + ((s + 1) & 1) * kActBytes;

    if constexpr (kRefill) {
      if constexpr (kU2 < kS) copy_table_set(lg, kU2);
      else copy_table_set(lg + 1, kU2 - kS);
    }
    if constexpr (kXNext) load_x(lg + 1, xnext);
    if constexpr (kNext) {
      if constexpr (kNJ == 0) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int t = 0; t < kX; ++t) xcur[rb][t] = xnext[rb][t];
      }
      prepare<kNJ>(st, xcur);
    }
    wait_vmcnt<0>();          // the table set and x have landed
    barrier_no_vm_drain();    // A(s+1)
  }

  template <bool kLast, int... kJs>
  __device__ __forceinline__ void group_steps(int lg, float (&xcur)[2][kX], float (&xnext)[2][kX],
                                              std::integer_sequence<int, kJs...>) const {
    (step<kLast, kJs>(lg, xcur, xnext), ...);
  }

  __device__ void run() const {
    float xcur[2][kX], xnext[2][kX];
    // Prologue: step 0's two planes, the table sets of the first group's spline steps 0 and
    // 1, its x, and step 0's activations (silu); A(0) publishes them.
    copy_table_set(0, 0);
    if (kS > 1) copy_table_set(0, 1);
    load_x(0, xcur);
    wait_vmcnt<0>();
    prepare<0>(smem + kActAt, xcur);
    barrier_no_vm_drain();  // A(0)
    for (int lg = 0; lg + 1 < nlg; ++lg) group_steps<false>(lg, xcur, xnext, std::make_integer_sequence<int, kQ>{});
    group_steps<true>(nlg - 1, xcur, xnext, std::make_integer_sequence<int, kQ>{});
  }
};

// Consumer phases.  A consumer lane (column fr of block cb, quarter fq) holds its weight
// fragments in registers: k = 8 fq .. 8 fq + 7 of each 32-k chunk (the sparse B operand
// takes two chunks, k and k + 32 of the step).  They come straight from the packed planes
// (one 1 KiB load per column block and chunk: 16 rows of 64 bytes); each consumer wave is
// the only reader of its 64 columns, so the weights bypass the LDS.  Activation fragments
// of two row blocks are read during the previous pair's MFMAs.
typedef _Float16 f16x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f16x16 join16(f16x8 a, f16x8 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
}

struct ActPair {
  f16x8 h[2], l[2];
  int idx[2];
};

template <bool kLo>
__device__ __forceinline__ void read_act(const uint8_t* ast, int lane, int rb, ActPair& a) {
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    a.h[r] = __builtin_bit_cast(f16x8, *reinterpret_cast<const i32x4*>(ast + (((rb + r) * 2 + 0) * 64 + lane) * 16));
    if constexpr (kLo)
      a.l[r] = __builtin_bit_cast(f16x8, *reinterpret_cast<const i32x4*>(ast + (((rb + r) * 2 + 1) * 64 + lane) * 16));
  }
  const i32x2 ix = *reinterpret_cast<const i32x2*>(ast + kActFragBytes + ((rb / 2) * 64 + lane) * 8);
  a.idx[0] = ix.x;
  a.idx[1] = ix.y;
}

// Phase L (kH false: hi_a * lo_w) or H (hi_a * hi_w, then lo_a * hi_w) of one step, with the
// weight plane in w0 / w1, the activations in `ast` and the first pair's already in `cur`.
// `load(k)` (k = 0 .. 3) loads column block k of another plane; the phase issues all four
// at its start, so they have the whole phase to land.  During its last pair, phase H reads
// phase L's first pair into `lfirst`; phase L, once that pair's activations are in
// registers, arrives at A(s+1) and then reads the next step's first pair (stage
// `ast_next`, just published) into `lfirst`.  The first pair's schedule places the
// phase's loads after its first MFMA and LDS read (measured about 1 % faster than before
// them).
template <bool kSparse, bool kH, typename Load>
__device__ __forceinline__ void consume_phase(const f16x8 (&w0)[kCB], const f16x8 (&w1)[kCB], const uint8_t* ast,
                                              int lane, f32x4 (&acc)[kRB][kCB], Load load, ActPair cur,
                                              ActPair& lfirst, const uint8_t* ast_next = nullptr) {
  constexpr int kTerms = kH ? 2 : 1;
  constexpr int kReads = kH ? 5 : 3;  // LDS reads of a pair
  load(0);
  load(1);
  load(2);
  load(3);
#pragma unroll
  for (int rb = 0; rb < kRB; rb += 2) {
    if constexpr (!kH) {
      if (rb + 2 == kRB) barrier_no_vm_drain();  // A(s+1): this pair's activations are in registers
    }
    ActPair nxt;
    if (rb + 2 < kRB) read_act<kH>(ast, lane, rb + 2, nxt);
    else if constexpr (kH) read_act<false>(ast, lane, 0, lfirst);
    else read_act<true>(ast_next, lane, 0, lfirst);
#pragma unroll
    for (int term = 0; term < kTerms; ++term)
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb) {
          const f16x8 a = term == 0 ? cur.h[r] : cur.l[r];
          if constexpr (kSparse)
            acc[rb + r][cb] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(a, join16(w0[cb], w1[cb]), acc[rb + r][cb],
                                                                       cur.idx[r], 0, 0);
          else
            acc[rb + r][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, w0[cb], acc[rb + r][cb], 0, 0, 0);
        }
    if (rb + 2 < kRB) {
#pragma unroll
      for (int u = 0; u < kReads; ++u) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                        // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                        // 1 LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 8 * kTerms / kReads - 1, 0);  // MFMAs
        if (u == 0) __builtin_amdgcn_sched_group_barrier(0x020, 8, 0);  // the loads
      }
    } else if constexpr (kH) {
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                        // 1 LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * kTerms, 0);               // MFMAs
        if (u == 0 || u == 2) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // empty load slot (kept: measured faster)
      }
    } else {
#pragma unroll
      for (int u = 0; u < 5; ++u) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                        // 1 LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                        // MFMA
        if (u == 0 || u == 3) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // empty load slot (kept: measured faster)
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (rb + 2 < kRB) cur = nxt;
  }
}

template <int kCp>
struct Consumer {
  static constexpr int kS = kCp / 2;
  static constexpr int kQ = 1 + kS;
  static constexpr int kChunksPerGroup = 1 + kCp;

  // Column block cb of this wave's fragments of plane rp, for the step at position kJ of
  // group lg (w1: the step's second chunk, spline steps only).
  template <int kJ>
  __device__ __forceinline__ void load_block(__amdgpu_buffer_rsrc_t rp, int lg, int cb, f16x8 (&w0)[kCB],
                                             f16x8 (&w1)[kCB]) const {
    const int q = (g0 + lg) * kChunksPerGroup + (kJ == 0 ? 0 : 2 * kJ - 1);
    const int so = q * Opad * 64;
    w0[cb] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rp, voff + cb * 1024, so, 0));
    if constexpr (kJ > 0)
      w1[cb] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rp, voff + cb * 1024, so + Opad * 64, 0));
  }

  // Step s = lg * kQ + kJ: phase H from hi(s) (in h0 / h1) while lo(s) loads into l0 / l1,
  // then phase L from lo(s) while hi(s+1) loads into h0 / h1, with A(s+1) before phase L's
  // last pair.  `first` holds step s's first activation pair on entry and step s+1's on
  // exit.  After the last step the hi loads re-read the current group and the last pair
  // reads the other stage (both harmless), so every step has the same shape.
  template <int kJ>
  __device__ __forceinline__ void step(int lg, int lane, f32x4 (&acc)[kRB][kCB], f16x8 (&h0)[kCB], f16x8 (&h1)[kCB],
                                       f16x8 (&l0)[kCB], f16x8 (&l1)[kCB], ActPair& first) const {
    const int s = lg * kQ + kJ;
    constexpr int kNJ = (kJ + 1) % kQ;
    const bool next = kJ + 1 < kQ || lg + 1 < nlg;
    const int lgn = kJ + 1 < kQ ? lg : (next ? lg + 1 : lg);
    const uint8_t* ast = smem + kActAt + (s & 1) * kActBytes;
    ActPair lfirst;
    consume_phase<(kJ > 0), true>(h0, h1, ast, lane, acc, [&](int k) { load_block<kJ>(rlo, lg, k, l0, l1); }, first,
                                  lfirst);
    consume_phase<(kJ > 0), false>(l0, l1, ast, lane, acc, [&](int k) { load_block<kNJ>(rhi, lgn, k, h0, h1); },
                                   lfirst, first, smem + kActAt + ((s + 1) & 1) * kActBytes);
  }

  template <int... kJs>
  __device__ __forceinline__ void group(int lg, int lane, f32x4 (&acc)[kRB][kCB], f16x8 (&h0)[kCB],
                                        f16x8 (&h1)[kCB], f16x8 (&l0)[kCB], f16x8 (&l1)[kCB], ActPair& first,
                                        std::integer_sequence<int, kJs...>) const {
    (step<kJs>(lg, lane, acc, h0, h1, l0, l1, first), ...);
  }

  uint8_t* smem;
  __amdgpu_buffer_rsrc_t rhi, rlo;
  int g0, nlg, Opad;
  int voff;  // this lane's fragment in a chunk: row n0 + 64 wave + fr, bytes 16 fq ..
};

// Output of a consumer accumulator: consumer wave wq, row block rb, column block cb, lane
// lq hold output column n0 + 64 wq + 16 cb + lq % 16 of batch rows m0 + 16 rb + 4 (lq / 16)
// + 0..3, scaled back by the column's scale.
__device__ __forceinline__ void store_slot(f32x4 val, int wq, int rb, int cb, int lq, int m0, int n0, int B, int O,
                                           const float* __restrict__ colscale, __amdgpu_buffer_rsrc_t ro) {
  const int o = n0 + wq * (kCB * 16) + cb * 16 + lq % 16;
  const float sc = colscale[o];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int row = m0 + rb * 16 + 4 * (lq / 16) + e;
    const unsigned off = (row < B && o < O) ? (unsigned)(((size_t)row * O + o) * 4) : kOutOfRange;
    // Through a scalar: hipcc turned __builtin_bit_cast(unsigned, val[e]) into a store of
    // element 0 for every e.
    const float ve = val[e] * sc;
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(ve), ro, off, 0, 0);
  }
}

// Split-K handover, all 512 threads: after every consumer has written its partial, thread 0
// releases them at agent scope and arrives on the tile's counter; the tile's last arrival
// sums the nsplit partials of every slot in split order (so the result does not depend on
// which split arrives last), 16 slots per thread with each split's loads in flight
// together, resets the counter and writes the output.  (Giving each wave 16 consecutive
// slot rows, so both 64-byte halves of an output line leave from one wave, measured about
// 1 us slower per call at the reference's timed shape.)
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
  constexpr int kTileSlots = BM * BN / 4;        // 16-byte slots per tile
  constexpr int kPer = kTileSlots / kThreads;    // per thread
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
    store_slot(sum[u], wq, rb, cb, lq, m0, n0, B, O, colscale, ro);
  }
}

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
  constexpr int kQ = 1 + kCp / 2;
  const int tm = (B + BM - 1) / BM, tn = Opad / BN;
  const int split = blockIdx.x % nsplit, tile = blockIdx.x / nsplit;
  const int g0 = split * gper, g1 = min(ngroups, g0 + gper);
  const int nlg = g1 - g0;
  int mt, nt;
  tile_of(tile, tm, tn, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);

  if (wave >= kConsumerWaves) {
    {
      Producer<kCp, kVec> p;
      p.smem = smem;
      p.I = I; p.L = L; p.B = B;
      p.g0 = g0; p.nlg = nlg;
      p.lane = lane; p.fr = lane % 16; p.fq = lane / 16; p.pw = wave - kConsumerWaves;
      p.row[0] = m0 + 32 * p.pw + p.fr;
      p.row[1] = p.row[0] + 16;
      p.tgb = tbl_group_bytes(L);
      p.rx = make_rsrc(x, (size_t)B * I * 4);
      p.rt = make_rsrc(tables, (size_t)ngroups * p.tgb);
      bool ok = true, card = true;
      for (int i = lane; i < nflags; i += kWave) {
        ok = ok && (uflags[i] & 1) != 0;
        card = card && (uflags[i] & 2) != 0;
      }
      p.uniform = __builtin_amdgcn_ballot_w64(!ok) == 0;
      p.cardinal = __builtin_amdgcn_ballot_w64(!card) == 0;
      p.C = L - 1 - kOrder;
      p.run();
    }
    wait_vmcnt<0>();  // no copy may still be writing LDS past this point
    if (nsplit > 1) split_k_finish(smem, tid, split, nsplit, tile, m0, n0, B, O, colscale, out, partial, counters);
    return;
  }

  f32x4 acc[kRB][kCB];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  Consumer<kCp> cons;
  cons.smem = smem;
  {
    const size_t wbytes = (size_t)ngroups * (1 + kCp) * Opad * kChunk * 2;
    cons.rhi = make_rsrc(bhi, wbytes);
    cons.rlo = make_rsrc(blo, wbytes);
  }
  cons.g0 = g0;
  cons.nlg = nlg;
  cons.Opad = Opad;
  cons.voff = (n0 + wave * (kCB * 16) + lane % 16) * 64 + 16 * (lane / 16);
  f16x8 h0[kCB], h1[kCB], l0[kCB], l1[kCB];
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb) cons.template load_block<0>(cons.rhi, 0, cb, h0, h1);  // hi(0)
  barrier_no_vm_drain();  // A(0)
  ActPair first;
  read_act<true>(smem + kActAt, lane, 0, first);
  for (int lg = 0; lg < nlg; ++lg)
    cons.group(lg, lane, acc, h0, h1, l0, l1, first, std::make_integer_sequence<int, kQ>{});
  wait_vmcnt<0>();  // the last step's (unused) loads

  if (nsplit > 1) {
    // This thread's 16-byte slots of the partial tile: (wave, rb, cb, lane), so every
    // store instruction of a wave covers 1 KiB of contiguous memory.  The stores are
    // system-scope (sc0 sc1: written through the L2), so the agent-scope release before the
    // arrival finds little dirty data in this XCD's L2 to write back; ordering is still the
    // fences' (split_k_finish).  Same bits; at the reference's timed shape (64 tiles, 4
    // splits) 75.4-75.9 -> 71.3-72.7 us per call (A/B on one box, both orders).
    const int tiles = gridDim.x / nsplit;
    float* mine = partial + ((size_t)split * tiles + tile) * (BM * BN);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(mine, (size_t)BM * BN * 4);
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, acc[rb][cb]), rp,
                                               (unsigned)((((wave * kRB + rb) * kCB + cb) * kWave + lane) * 16), 0,
                                               kStoreSystem);
    split_k_finish(smem, tid, split, nsplit, tile, m0, n0, B, O, colscale, out, partial, counters);
    return;
  }

  // Epilogue.  Each accumulator holds one column of 4 rows, so a store instruction writes
  // 64-byte halves of 4 output lines; the wave's four column blocks of a row go out back to
  // back, so both halves of each line leave in consecutive instructions.  Same bits; A/B on
  // one box (BASELINE): 258.3 against 260.4 us per call with the column blocks outermost.
  // Staging each row block in LDS to store 256-byte row segments measured the same (258.2).
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(out, (size_t)B * O * 4);
  const int fr = lane % 16, fq = lane / 16;
  float csc[kCB];
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb) csc[cb] = colscale[n0 + wave * (kCB * 16) + cb * 16 + fr];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) {
        const int row = m0 + rb * 16 + 4 * fq + e, o = n0 + wave * (kCB * 16) + cb * 16 + fr;
        const unsigned off = (row < B && o < O) ? (unsigned)(((size_t)row * O + o) * 4) : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[rb][cb][e] * csc[cb]), ro, off, 0, 0);
      }
}

}  // namespace kan
}  // namespace taskops
