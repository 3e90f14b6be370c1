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
//           chunks of a segment of kWaves*kSeg chunks and publishes the composed map of
//           its span in LDS; a shuffle scan over those kWaves records gives each wave the
//           value flowing into its span from the spans after it.
// Segments are walked from the row end toward its start with a running carry.  Rows are
// independent workgroups, so thousands of them stream through the CUs staggered: loads,
// scans and stores of different rows overlap.  The wave and workgroup scans and the carries
// between lanes, chunks, waves and segments are fp64.  A lane's own 4 steps run in fp32: its
// map's R in pass 1, and in pass 2 the 3 steps after the first, which starts from the fp64
// carry.  That adds at most ~2e-7 relative per output (about 1e-6 absolute where terms
// cancel), against the op's atol = rtol = 1e-5, and measured 1.5-2 % faster than fp64
// throughout.  Pass 1 also keeps, for each of a wave's chunks, the composed map of the
// wave's later chunks (wave-uniform, in scalar registers), so in pass 2 every chunk's
// incoming value is one fp64 fma of the wave's incoming value and the chunks do not wait on
// each other; the wave scan's span factors g^(4 * 2^i) are computed once per workgroup.
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
template <int kStorePolicy>  // bit 0 sc0, bit 1 nt
__device__ __forceinline__ void store_row16(float* row_base, int T, int t, f32x4 w) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(row_base, (short)0, T * 4, 0x00020000);
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
  static_assert(kPerLane % 4 == 0, "lanes own whole 16-byte reward vectors");
  constexpr int kChunk = kWave * kPerLane;
  constexpr int kQ = kPerLane / 4;
  __shared__ double span_a[kWaves], span_r[kWaves];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int nchunks = (T + kChunk - 1) / kChunk;

  // gk = g^kPerLane, and pw_rest = g^(kPerLane*(63-lane)) (the A of lanes lane+1..63 with
  // no done step), by repeated squaring.
  double gk = 1.0;
#pragma unroll
  for (int e = 0; e < kPerLane; ++e) gk *= g;
  // gpow[i] = g^(kPerLane * 2^i): the wave scan's span factors, the same products as
  // squaring per step, computed once.
  double gpow[7];
  gpow[0] = gk;
#pragma unroll
  for (int i = 1; i < 7; ++i) gpow[i] = gpow[i - 1] * gpow[i - 1];
  double pw_rest = 1.0;
  {
    double base = gk;
    for (int e = kWave - 1 - lane; e > 0; e >>= 1) {
      if (e & 1) pw_rest *= base;
      base *= base;
    }
  }
  const float gf = (float)g;
  const int row = blockIdx.x;
  const size_t base = (size_t)row * (size_t)T;
  const float* rr = reward + base;
  const uint8_t* dd = done + base;
  float* oo = out + base;
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
            const f32x4 v = (kNT & 1) ? __builtin_nontemporal_load(src) : *src;
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

    // Lane maps and wave suffix scans.  A map is (R, A): v -> R + A*v.  A lane's A over its
    // kPerLane steps is 0 if one of them is a done step, else g^kPerLane; in the suffix
    // scan every combining lane's span is exactly kPerLane*off steps, so its A is 0 or the
    // wave-uniform g^(kPerLane*off).  A therefore travels as one bit per lane in a 64-bit
    // ballot mask (bit L: a done step in lanes L.. of the span), and only R is a per-lane
    // double.  A chunk's total map is lane 0's.  Steps past the row end hold r = 0 and no
    // done, so they only ever multiply the zero carry of the row end.
    double sr[kSeg];
    unsigned long long smask[kSeg];
    double wr = 0.0, wa = 1.0;  // this wave's span map
    double after_r[kSeg], after_a[kSeg];  // map of this wave's chunks after chunk c
#pragma unroll
    for (int c = kSeg - 1; c >= 0; --c) {
      float Rf = 0.0f;
#pragma unroll
      for (int e = kPerLane - 1; e >= 0; --e) Rf = fmaf(coef32(dn[c][e / 4], e % 4, gf), Rf, r[c][e]);
      double R = (double)Rf;
      unsigned any = 0u;
#pragma unroll
      for (int q = 0; q < kQ; ++q) any |= dn[c][q];
      unsigned long long mask = __ballot(any != 0u);
#pragma unroll
      for (int lv = 0, off = 1; off < kWave; ++lv, off <<= 1) {
        const double Rn = __shfl_down(R, off, kWave);
        const bool blocked = (mask >> lane) & 1ull;
        if (lane + off < kWave && !blocked) R = fma(gpow[lv], Rn, R);
        mask |= mask >> off;
      }
      const double G = gpow[6];  // g^(kPerLane*64)
      sr[c] = R;
      smask[c] = mask;
      after_r[c] = uniform(wr);
      after_a[c] = uniform(wa);
      if (c0 + c < hi) {
        const double cr = __shfl(R, 0, kWave);
        const double ca = (mask & 1ull) ? 0.0 : G;  // G is now g^(kPerLane*64)
        wr = fma(ca, wr, cr);
        wa = ca * wa;
      }
    }
    if (lane == 0) {
      span_r[wave] = wr;
      span_a[wave] = wa;
    }
    __syncthreads();
    // Lane v holds span v; a suffix scan over the kWaves lanes composes spans v.. so that
    // lane v holds the map from span v's start to the segment end.
    double sa_v = lane < kWaves ? span_a[lane] : 1.0, sr_v = lane < kWaves ? span_r[lane] : 0.0;
#pragma unroll
    for (int off = 1; off < kWaves; off <<= 1) {
      const double Rn = __shfl_down(sr_v, off, kWave), An = __shfl_down(sa_v, off, kWave);
      if (lane + off < kWaves) {
        sr_v = fma(sa_v, Rn, sr_v);
        sa_v = sa_v * An;
      }
    }
    // Value flowing into this wave's span from the later spans, and into the segment.
    const double cin_a = __shfl(sa_v, wave + 1, kWave), cin_r = __shfl(sr_v, wave + 1, kWave);
    double cin = wave + 1 < kWaves ? fma(cin_a, carry, cin_r) : carry;
    const double next_carry = fma(__shfl(sa_v, 0, kWave), carry, __shfl(sr_v, 0, kWave));

#pragma unroll
    for (int c = kSeg - 1; c >= 0; --c) {
      if (c0 + c >= hi) continue;
      const int t0 = (c0 + c) * kChunk + lane * kPerLane;
      // Keep only the raw floats and done words live across the scan: without this the
      // compiler holds the first pass's fp64 conversions and coefficients (32 VGPRs).
#pragma unroll
      for (int e = 0; e < kPerLane; ++e) asm volatile("" : "+v"(r[c][e]));
#pragma unroll
      for (int q = 0; q < kQ; ++q) asm volatile("" : "+v"(dn[c][q]));
      // Value entering this chunk (the wave's later chunks applied to cin), then entering
      // this lane's last step (lanes lane+1.. applied to it).
      const double cin_c = fma(after_a[c], cin, after_r[c]);
      const double Rn = __shfl_down(sr[c], 1, kWave);
      const bool later_done = lane + 1 < kWave && ((smask[c] >> (lane + 1)) & 1ull);
      const double An = later_done ? 0.0 : pw_rest;
      const double vin = (lane == kWave - 1) ? cin_c : fma(An, cin_c, Rn);
      float o[kPerLane];
      // The lane's last step from the fp64 value entering it, the others in fp32.
      o[kPerLane - 1] = (float)fma(coef(dn[c][(kPerLane - 1) / 4], (kPerLane - 1) % 4, g), vin,
                                   (double)r[c][kPerLane - 1]);
#pragma unroll
      for (int e = kPerLane - 2; e >= 0; --e) o[e] = fmaf(coef32(dn[c][e / 4], e % 4, gf), o[e + 1], r[c][e]);
#pragma unroll
      for (int q = 0; q < kQ; ++q) {
        const int t = t0 + 4 * q;
        if constexpr (kVec) {
          if (t < T) {
            const f32x4 w = {o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
            if constexpr (((kNT >> 1) & 3) != 0)
              store_row16<(kNT >> 1) & 3>(oo, T, t, w);
            else
              *reinterpret_cast<f32x4*>(oo + t) = w;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (t + e < T) oo[t + e] = o[4 * q + e];
        }
      }

    }
    carry = next_carry;
    __syncthreads();  // span_* are rewritten by the next segment
  }
}

}  // namespace taskops
