// reward_to_go kernel template (instantiated by reward_to_go.hip).
//
// Op: tasks/reward_to_go/reference.py:34-42 (fp64 backward loop); prompt text
// tasks/reward_to_go/prompt.md ("output[b,t] = reward[b,t] + gamma * next").
//
// Each time step is the affine map  v -> r[t] + a[t] * v  with a[t] = done[t] ? 0 : gamma,
// and out[t] is the composition of the maps t..T-1 applied to 0.  Maps compose
// associatively, so a row is scanned hierarchically:
//   lane  — a lane owns kPerLane = 4 consecutive steps of each of its chunks (one 16-byte
//           reward vector, one 4-byte done word) and composes their maps serially;
//   wave  — a log-depth suffix scan of the 64 lane maps (6 shuffle steps) gives every
//           lane the map of the rest of its chunk of 256 steps; a wave's kSeg chunk scans
//           run interleaved, level by level, so their shuffles overlap;
//   workgroup — one workgroup owns one row; its kWaves waves each own kSeg consecutive
//           chunks of a segment of kWaves*kSeg chunks and publish the composed map of
//           their span in LDS; every lane then composes the spans after its wave's, one
//           fp64 fma each, to get the value flowing into its span.
// Segments are walked from the row end toward its start with a running carry.  Rows are
// independent workgroups, so thousands of them stream through the CUs staggered: loads,
// scans and stores of different rows overlap.
// Precision: a lane's 4-step map and the wave scan are fp32 (the scan's span factors
// g^(4 * 2^i) are fp64 powers rounded once); everything they feed — the compositions of
// chunks, spans and segments, each chunk's incoming value and the first of a lane's 4
// output steps — is fp64; the lane's 3 other output steps are fp32.  Measured worst error
// against the fp64 oracle: 0.16 of the op's atol = rtol = 1e-5 bound at BASELINE (gamma
// 0.99), 0.55 on gamma = 1 rows of U[-1, 1] rewards with no done step (rounding errors
// then never decay along the row; fp64 scans gave 0.064 and 0.28).  Against fp64 scans
// this measured 26.0 against 27.0 us per call at B = T = 4096.  Pass 1 also keeps, for
// each of a wave's chunks, the composed map of the wave's later chunks (wave-uniform, in
// scalar registers), so in pass 2 every chunk's incoming value is one fp64 fma of the
// wave's incoming value and the chunks do not wait on each other.
// HBM-bound: 9 algorithmic bytes per element (4 reward + 1 done + 4 out).
#pragma once

#include "common.hpp"

namespace taskops {

namespace rtg_detail {
using f32x4 = float __attribute__((ext_vector_type(4)));

// A wave-uniform double moved to scalar registers (it is the same in every lane).
__device__ __forceinline__ double uniform(double v) {
  const long long b = __double_as_longlong(v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)b);
  const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(b >> 32));
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

__device__ __forceinline__ double coef(unsigned word, int byte, double g) {
  return ((word >> (8 * byte)) & 0xFFu) ? 0.0 : g;
}
__device__ __forceinline__ float coef32(unsigned word, int byte, float g) {
  return ((word >> (8 * byte)) & 0xFFu) ? 0.0f : g;
}

// Output stores as buffer stores with an explicit cache policy.  Measured on MI355X at
// B = T = 4096 (80 MB read, 64 MB written): a plain copy of the same traffic takes 31.0 us
// with plain stores and 28.7 us with nt | sc0; policies with sc1 set take 51-68 us.  Which
// policy pays depends on the access pattern: with 4 steps per lane (whole 1 KiB per store
// instruction) nt stores are the fastest, with 8 steps per lane (every other 16 bytes)
// they are the slowest (reward_to_go.hip).
// The descriptor spans the row, so T * 4 bytes must fit its 32-bit size: the host takes
// rows of 2^30 steps or more down the element path.
template <int kStorePolicy>  // bit 0 sc0, bit 1 nt
__device__ __forceinline__ void store_row16(float* row_base, int T, int t, f32x4 w) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(row_base, (short)0, (int)((unsigned)T * 4u), 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, w), rs,
                                         (unsigned)t * 4u, 0, kStorePolicy);
}
}  // namespace rtg_detail

// kNT: bit 0 = non-temporal loads; bits 1-2 = the cache policy of buffer output stores
// (store_row16), 0 = plain stores.
template <int kWaves, int kPerLane, int kSeg, bool kVec, int kNT>
__global__ __launch_bounds__(kWaves * 64) void reward_to_go_kernel(
    const float* __restrict__ reward, const uint8_t* __restrict__ done, double g, int B, int T,
    float* __restrict__ out) {
  using namespace rtg_detail;
  static_assert(kPerLane == 4, "a lane owns one 16-byte reward vector per chunk");
  constexpr int kChunk = kWave * kPerLane;
  __shared__ double span_a[kWaves], span_r[kWaves];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int nchunks = (T + kChunk - 1) / kChunk;

  double gk = 1.0;
#pragma unroll
  for (int e = 0; e < kPerLane; ++e) gk *= g;
  double gpow[7];
  gpow[0] = gk;
#pragma unroll
  for (int i = 1; i < 7; ++i) gpow[i] = gpow[i - 1] * gpow[i - 1];
  float gpowf[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) gpowf[i] = (float)gpow[i];
  // gk = g^kPerLane; gpow[i] = g^(kPerLane * 2^i), the wave scan's span factors (fp64
  // powers, rounded once to fp32 for the scan); pw_rest = g^(kPerLane * (63 - lane)), the A
  // of lanes lane+1..63 with no done step.
  double pw_rest = 1.0;
  {
    double base = gk;
    for (int e = kWave - 1 - lane; e > 0; e >>= 1) {
      if (e & 1) pw_rest *= base;
      base *= base;
    }
  }
  const float gf = (float)g;
  const size_t base = (size_t)blockIdx.x * (size_t)T;
  const float* rr = reward + base;
  const uint8_t* dd = done + base;
  float* oo = out + base;
  double carry = 0.0;
  for (int hi = nchunks; hi > 0; hi -= kWaves * kSeg) {
    const int lo = hi > kWaves * kSeg ? hi - kWaves * kSeg : 0;
    const int c0 = lo + wave * kSeg;
    float r[kSeg][4];
    unsigned dn[kSeg];
#pragma unroll
    for (int c = 0; c < kSeg; ++c) {
      const int t = (c0 + c) * kChunk + lane * kPerLane;
      dn[c] = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[c][e] = 0.0f;
      if (c0 + c >= hi) continue;
      if constexpr (kVec) {
        if (t < T) {
          const f32x4* src = reinterpret_cast<const f32x4*>(rr + t);
          const f32x4 v = (kNT & 1) ? __builtin_nontemporal_load(src) : *src;
          r[c][0] = v.x;
          r[c][1] = v.y;
          r[c][2] = v.z;
          r[c][3] = v.w;
          dn[c] = *reinterpret_cast<const unsigned*>(dd + t);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (t + e < T) {
            r[c][e] = rr[t + e];
            dn[c] |= (unsigned)(dd[t + e] != 0) << (8 * e);
          }
        }
      }
    }

    // Lane maps and wave suffix scans.  A map is (R, A): v -> R + A*v.  A lane's A over its
    // 4 steps is 0 if one of them is a done step, else g^4; in the suffix scan every
    // combining lane's span is exactly 4*off steps, so its A is 0 or the wave-uniform
    // g^(4*off).  A therefore travels as one bit per lane in a 64-bit ballot mask (bit L: a
    // done step in lanes L.. of the span), and only R is a per-lane value.  A chunk's total
    // map is lane 0's.  Steps past the row end hold r = 0 and no done, so they only ever
    // multiply the zero carry of the row end.
    float R[kSeg];
    unsigned long long mask[kSeg];
#pragma unroll
    for (int c = 0; c < kSeg; ++c) {
      float Rf = 0.0f;
#pragma unroll
      for (int e = 3; e >= 0; --e) Rf = fmaf(coef32(dn[c], e, gf), Rf, r[c][e]);
      R[c] = Rf;
      mask[c] = __ballot(dn[c] != 0u);
    }
#pragma unroll
    for (int lv = 0, off = 1; off < kWave; ++lv, off <<= 1) {
#pragma unroll
      for (int c = 0; c < kSeg; ++c) {
        const float Rn = __shfl_down(R[c], off, kWave);
        const bool blocked = (mask[c] >> lane) & 1ull;
        if (lane + off < kWave && !blocked) R[c] = fmaf(gpowf[lv], Rn, R[c]);
        mask[c] |= mask[c] >> off;
      }
    }
    // This wave's span map (wr, wa) and, for each chunk, the map of the wave's chunks after
    // it (wave-uniform).
    const double G = gpow[6];  // g^256, a whole chunk with no done step
    double wr = 0.0, wa = 1.0;
    double after_r[kSeg], after_a[kSeg];
#pragma unroll
    for (int c = kSeg - 1; c >= 0; --c) {
      after_r[c] = uniform(wr);
      after_a[c] = uniform(wa);
      if (c0 + c < hi) {
        const double cr = (double)__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, R[c]), 0));
        const double ca = (mask[c] & 1ull) ? 0.0 : G;
        wr = fma(ca, wr, cr);
        wa = ca * wa;
      }
    }
    if (lane == 0) {
      span_r[wave] = wr;
      span_a[wave] = wa;
    }
    __syncthreads();
    // Compose the spans from the segment end: the value entering this wave's span, and the
    // value entering the segment (the next segment's carry).
    double x = carry, cin = carry;
#pragma unroll
    for (int v = kWaves - 1; v >= 0; --v) {
      if (v == wave) cin = x;
      x = fma(span_a[v], x, span_r[v]);
    }
    const double next_carry = x;

#pragma unroll
    for (int c = kSeg - 1; c >= 0; --c) {
      if (c0 + c >= hi) continue;
      const int t = (c0 + c) * kChunk + lane * kPerLane;
      // Keep only the raw floats and done words live across the scan: without this the
      // compiler holds the first pass's conversions and coefficients.
#pragma unroll
      for (int e = 0; e < 4; ++e) asm volatile("" : "+v"(r[c][e]));
      asm volatile("" : "+v"(dn[c]));
      // Value entering this chunk (the wave's later chunks applied to cin), then entering
      // this lane's last step (lanes lane+1.. applied to it).
      const double cin_c = fma(after_a[c], cin, after_r[c]);
      const double Rn = (double)__shfl_down(R[c], 1, kWave);
      const bool later_done = lane + 1 < kWave && ((mask[c] >> (lane + 1)) & 1ull);
      const double An = later_done ? 0.0 : pw_rest;
      const double vin = (lane == kWave - 1) ? cin_c : fma(An, cin_c, Rn);
      // The lane's last step from the fp64 value entering it, the others in fp32.
      float o[4];
      o[3] = (float)fma(coef(dn[c], 3, g), vin, (double)r[c][3]);
#pragma unroll
      for (int e = 2; e >= 0; --e) o[e] = fmaf(coef32(dn[c], e, gf), o[e + 1], r[c][e]);
      if constexpr (kVec) {
        if (t < T) {
          const f32x4 w = {o[0], o[1], o[2], o[3]};
          if constexpr (((kNT >> 1) & 3) != 0)
            store_row16<(kNT >> 1) & 3>(oo, T, t, w);
          else
            *reinterpret_cast<f32x4*>(oo + t) = w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (t + e < T) oo[t + e] = o[e];
      }
    }
    carry = next_carry;
    __syncthreads();  // span_* are rewritten by the next segment
  }
}

}  // namespace taskops
