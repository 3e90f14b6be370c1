// reward_to_go kernel template (instantiated by reward_to_go.hip).
//
// Op: tasks/reward_to_go/reference.py:34-42 (fp64 backward loop); prompt text
// tasks/reward_to_go/prompt.md ("output[b,t] = reward[b,t] + gamma * next").
//
// Each time step is the affine map  v -> r[t] + a[t] * v  with a[t] = done[t] ? 0 : gamma,
// and out[t] is the composition of the maps t..T-1 applied to 0.  Maps compose
// associatively, so a row is scanned hierarchically:
//   lane  — a lane owns kPerLane consecutive steps (16-byte reward vectors, 4-byte done
//           words) and composes their maps serially;
//   wave  — a log-depth suffix scan of the 64 lane maps (6 shuffle steps) gives every
//           lane the map of the rest of its chunk of 64*kPerLane steps;
//   workgroup — one workgroup owns one row; its kWaves waves each own kSeg consecutive
//           chunks of a segment of kWaves*kSeg chunks, publish the composed map of their
//           span in LDS, and each derives the value flowing into its span from the spans
//           after it.
// Segments are walked from the row end toward its start with a running carry.  Rows are
// independent workgroups, so thousands of them stream through the CUs staggered: loads,
// scans and stores of different rows overlap.  Maps and carries are fp64; each output is
// rounded to fp32 once.
// HBM-bound: 9 algorithmic bytes per element (4 reward + 1 done + 4 out).
#pragma once

#include "common.hpp"

namespace taskops {

namespace rtg_detail {
using f32x4 = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ double coef(unsigned word, int byte, double g) {
  return ((word >> (8 * byte)) & 0xFFu) ? 0.0 : g;
}
}  // namespace rtg_detail

template <int kWaves, int kPerLane, int kSeg, bool kVec, bool kNT>
__global__ __launch_bounds__(kWaves * 64) void reward_to_go_kernel(
    const float* __restrict__ reward, const uint8_t* __restrict__ done, double g, int B, int T,
    float* __restrict__ out) {
  using namespace rtg_detail;
  static_assert(kPerLane % 4 == 0, "lanes own whole 16-byte reward vectors");
  constexpr int kChunk = kWave * kPerLane;
  constexpr int kQ = kPerLane / 4;
  __shared__ double span_a[kWaves], span_r[kWaves];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int row = blockIdx.x;
  const size_t base = (size_t)row * (size_t)T;
  const float* rr = reward + base;
  const uint8_t* dd = done + base;
  float* oo = out + base;
  const int nchunks = (T + kChunk - 1) / kChunk;

  double carry = 0.0;  // value of the step after the current segment (0 past the row end)
  for (int hi = nchunks; hi > 0; hi -= kWaves * kSeg) {
    const int lo = hi > kWaves * kSeg ? hi - kWaves * kSeg : 0;
    const int c0 = lo + wave * kSeg;  // this wave's chunks: [c0, c0 + kSeg) within [lo, hi)
    float r[kSeg][kPerLane];
    unsigned dn[kSeg][kQ];
#pragma unroll
    for (int c = 0; c < kSeg; ++c) {
      const int t0 = (c0 + c) * kChunk + lane * kPerLane;
#pragma unroll
      for (int q = 0; q < kQ; ++q) dn[c][q] = 0u;
#pragma unroll
      for (int e = 0; e < kPerLane; ++e) r[c][e] = 0.0f;
      if (c0 + c >= hi) continue;
#pragma unroll
      for (int q = 0; q < kQ; ++q) {
        const int t = t0 + 4 * q;
        if constexpr (kVec) {
          if (t < T) {
            const f32x4* src = reinterpret_cast<const f32x4*>(rr + t);
            const f32x4 v = kNT ? __builtin_nontemporal_load(src) : *src;
            r[c][4 * q + 0] = v.x;
            r[c][4 * q + 1] = v.y;
            r[c][4 * q + 2] = v.z;
            r[c][4 * q + 3] = v.w;
            dn[c][q] = *reinterpret_cast<const unsigned*>(dd + t);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (t + e < T) {
              r[c][4 * q + e] = rr[t + e];
              dn[c][q] |= (unsigned)(dd[t + e] != 0) << (8 * e);
            }
          }
        }
      }
    }

    // Lane maps and wave suffix scans; a chunk's total map is lane 0's.  Steps past the
    // row end hold r = 0, so they only ever multiply the zero carry of the row end.
    double sr[kSeg], sa[kSeg];
    double wr = 0.0, wa = 1.0;  // this wave's span map
#pragma unroll
    for (int c = kSeg - 1; c >= 0; --c) {
      double R = 0.0, A = 1.0;
#pragma unroll
      for (int e = kPerLane - 1; e >= 0; --e) {
        const double a = coef(dn[c][e / 4], e % 4, g);
        R = fma(a, R, (double)r[c][e]);
        A = a * A;
      }
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const double Rn = __shfl_down(R, off, kWave);
        const double An = __shfl_down(A, off, kWave);
        if (lane + off < kWave) {
          R = fma(A, Rn, R);
          A = A * An;
        }
      }
      sr[c] = R;
      sa[c] = A;
      if (c0 + c < hi) {
        const double cr = __shfl(R, 0, kWave), ca = __shfl(A, 0, kWave);
        wr = fma(ca, wr, cr);
        wa = ca * wa;
      }
    }
    if (lane == 0) {
      span_r[wave] = wr;
      span_a[wave] = wa;
    }
    __syncthreads();
    double cin = carry;  // value flowing into this wave's span from the later spans
    for (int v = kWaves - 1; v > wave; --v) cin = fma(span_a[v], cin, span_r[v]);
    double next_carry = carry;
    for (int v = kWaves - 1; v >= 0; --v) next_carry = fma(span_a[v], next_carry, span_r[v]);

#pragma unroll
    for (int c = kSeg - 1; c >= 0; --c) {
      if (c0 + c >= hi) continue;
      const int t0 = (c0 + c) * kChunk + lane * kPerLane;
      const double Rn = __shfl_down(sr[c], 1, kWave);
      const double An = __shfl_down(sa[c], 1, kWave);
      double v = (lane == kWave - 1) ? cin : fma(An, cin, Rn);
      float o[kPerLane];
#pragma unroll
      for (int e = kPerLane - 1; e >= 0; --e) {
        v = fma(coef(dn[c][e / 4], e % 4, g), v, (double)r[c][e]);
        o[e] = (float)v;
      }
#pragma unroll
      for (int q = 0; q < kQ; ++q) {
        const int t = t0 + 4 * q;
        if constexpr (kVec) {
          if (t < T) {
            const f32x4 w = {o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
            f32x4* dst = reinterpret_cast<f32x4*>(oo + t);
            if constexpr (kNT)
              __builtin_nontemporal_store(w, dst);
            else
              *dst = w;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (t + e < T) oo[t + e] = o[4 * q + e];
        }
      }
      cin = __shfl(v, 0, kWave);  // value at the chunk's first step
    }
    carry = next_carry;
    __syncthreads();  // span_* are rewritten by the next segment
  }
}

}  // namespace taskops
