// ppo_clip kernel template (instantiated by ppo_clip.hip).
//
// Op: tasks/ppo_clip/reference.py:27-39 (fp64 oracle :42-45, eps rounded to fp32 first).
// HBM-bound: 12 bytes per sample (16 with entropy).  Per sample, with lw = cur - old:
//   r = exp(lw); gain = A * (A > 0 && lw > log1p(eps) ? 1 + eps
//                         : A < 0 && lw < log1p(-eps) ? 1 - eps : r)
// which equals min(r*A, exp(clamp(lw, log1p(-eps), log1p(eps)))*A); the clip test runs on
// the exact fp64 difference against the fp64 bounds, so the clip count matches the fp64
// reference.  ESS uses exp(2 lse(lw) - lse(2 lw)) / N = (sum r)^2 / (N sum r^2).
// Per-thread sums are fp32 over one unrolled iteration, then fp64; each workgroup
// publishes a 7-field record and the last one to arrive combines the records in a fixed
// order (common.hpp), so repeated calls give identical bits.
#pragma once

#include "common.hpp"

namespace taskops {

constexpr int kPpoFields = 7;  // gain, clipped, kl, sum r, sum r^2, sum entropy, max r

struct PpoWorkspace {
  static constexpr int kMaxBlocks = 4096;
  double partial[kMaxBlocks][8];
  Arrivals arrivals;
};

struct PpoParams {
  double lo, hi;     // log1p(-eps), log1p(eps) in fp64
  float lo_ratio;    // 1 - eps
  float hi_ratio;    // 1 + eps
};

namespace ppo_detail {

using f32x4 = float __attribute__((ext_vector_type(4)));

template <bool kNT>
__device__ __forceinline__ f32x4 ld(const f32x4* p) {
  if constexpr (kNT) return __builtin_nontemporal_load(p);
  return *p;
}

struct Acc {
  float gain = 0.f, kl = 0.f, sr = 0.f, sr2 = 0.f, se = 0.f, maxr = 0.f;
  unsigned clipped = 0;
};

__device__ __forceinline__ void sample(Acc& s, float cur, float old, float adv, const PpoParams& p) {
  const float lw = cur - old;
  const double lwd = (double)cur - (double)old;
  const float r = expf(lw);
  const bool below = lwd < p.lo, above = lwd > p.hi;
  const float ratio = (adv > 0.f && above) ? p.hi_ratio : ((adv < 0.f && below) ? p.lo_ratio : r);
  s.gain += ratio * adv;
  s.clipped += (unsigned)(below | above);
  s.kl += (r - 1.0f) - lw;
  s.sr += r;
  s.sr2 += r * r;
  s.maxr = fmaxf(s.maxr, r);
}

struct Totals {
  double gain = 0, clipped = 0, kl = 0, sr = 0, sr2 = 0, se = 0;
  float maxr = 0.f;
  __device__ void fold(const Acc& a) {
    gain += a.gain;
    clipped += (double)a.clipped;
    kl += a.kl;
    sr += a.sr;
    sr2 += a.sr2;
    se += a.se;
    maxr = fmaxf(maxr, a.maxr);
  }
};

}  // namespace ppo_detail

template <int kThreads, int kUnroll, bool kVec, bool kEntropy, bool kNT>
__global__ __launch_bounds__(kThreads) void ppo_clip_kernel(
    int64_t n, const float* __restrict__ cur, const float* __restrict__ old,
    const float* __restrict__ adv, const float* __restrict__ ent, PpoParams p, float coef,
    double (*__restrict__ records)[8], Arrivals* __restrict__ arrivals, float* __restrict__ out) {
  using namespace ppo_detail;
  constexpr int kFields = kPpoFields;
  __shared__ double lds[kFields][kThreads / kWave];
  __shared__ bool last;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const int64_t tid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  Totals tot;
  if constexpr (kVec) {
    const f32x4* c4 = reinterpret_cast<const f32x4*>(cur);
    const f32x4* o4 = reinterpret_cast<const f32x4*>(old);
    const f32x4* a4 = reinterpret_cast<const f32x4*>(adv);
    const f32x4* e4 = reinterpret_cast<const f32x4*>(ent);
    const int64_t n4 = n >> 2;
    int64_t i = tid;
    for (; i + (kUnroll - 1) * stride < n4; i += kUnroll * stride) {
      f32x4 c[kUnroll], o[kUnroll], a[kUnroll], e[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        c[u] = ld<kNT>(c4 + i + u * stride);
        o[u] = ld<kNT>(o4 + i + u * stride);
        a[u] = ld<kNT>(a4 + i + u * stride);
        if constexpr (kEntropy) e[u] = ld<kNT>(e4 + i + u * stride);
      }
      Acc s;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        sample(s, c[u].x, o[u].x, a[u].x, p);
        sample(s, c[u].y, o[u].y, a[u].y, p);
        sample(s, c[u].z, o[u].z, a[u].z, p);
        sample(s, c[u].w, o[u].w, a[u].w, p);
        if constexpr (kEntropy) s.se += (e[u].x + e[u].y) + (e[u].z + e[u].w);
      }
      tot.fold(s);
    }
    for (; i < n4; i += stride) {
      Acc s;
      const f32x4 c = ld<kNT>(c4 + i), o = ld<kNT>(o4 + i), a = ld<kNT>(a4 + i);
      sample(s, c.x, o.x, a.x, p);
      sample(s, c.y, o.y, a.y, p);
      sample(s, c.z, o.z, a.z, p);
      sample(s, c.w, o.w, a.w, p);
      if constexpr (kEntropy) {
        const f32x4 e = ld<kNT>(e4 + i);
        s.se += (e.x + e.y) + (e.z + e.w);
      }
      tot.fold(s);
    }
    if (tid < (n & 3)) {
      const int64_t k = (n4 << 2) + tid;
      Acc s;
      sample(s, cur[k], old[k], adv[k], p);
      if constexpr (kEntropy) s.se += ent[k];
      tot.fold(s);
    }
  } else {
    for (int64_t k = tid; k < n; k += stride) {
      Acc s;
      sample(s, cur[k], old[k], adv[k], p);
      if constexpr (kEntropy) s.se += ent[k];
      tot.fold(s);
    }
  }

  // Workgroup reduction of the seven fields (fixed order; max is order-free).
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  double v[kFields] = {tot.gain, tot.clipped, tot.kl, tot.sr, tot.sr2, tot.se, (double)tot.maxr};
#pragma unroll
  for (int f = 0; f < kFields - 1; ++f) v[f] = wave_sum(v[f]);
  v[kFields - 1] = (double)wave_max(tot.maxr);
  if (lane == 0) {
#pragma unroll
    for (int f = 0; f < kFields; ++f) lds[f][wave] = v[f];
  }
  __syncthreads();
  double rec[kFields];
#pragma unroll
  for (int f = 0; f < kFields; ++f) {
    double t = lds[f][0];
    for (int w = 1; w < kThreads / kWave; ++w)
      t = (f == kFields - 1) ? fmax(t, lds[f][w]) : t + lds[f][w];
    rec[f] = t;
  }
  if (!publish_and_arrive<kFields>(records[blockIdx.x], rec, arrivals, &last)) return;

  // Finishing workgroup: wave w reduces fields w, w + waves, ... over all records (ratios
  // are positive, so 0 is the identity of the max as well as of the sums).
  __syncthreads();
  for (int f = wave; f < kFields; f += kThreads / kWave) {
    double t = (f == kFields - 1) ? gather_records<true>(&records[0][f], 8, (int)gridDim.x, lane, kWave)
                                  : gather_records<false>(&records[0][f], 8, (int)gridDim.x, lane, kWave);
    if (f == kFields - 1) {
#pragma unroll
      for (int off = kWave / 2; off > 0; off >>= 1) t = fmax(t, __shfl_xor(t, off, kWave));
    } else {
      t = wave_sum(t);
    }
    if (lane == 0) lds[f][0] = t;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const double nd = (double)n;
    const double gain = lds[0][0], clipped = lds[1][0], kl = lds[2][0], sr = lds[3][0],
                 sr2 = lds[4][0], se = lds[5][0], maxr = lds[6][0];
    out[0] = (float)(-gain / nd);
    out[1] = (float)(clipped / nd);
    out[2] = (float)(kl / nd);
    out[3] = (float)((sr / nd) * (sr / sr2));
    out[4] = (float)maxr;
    out[5] = (float)(sr / nd);
    if constexpr (kEntropy) {
      const double me = se / nd;
      out[6] = (float)me;
      out[7] = (float)(-(double)coef * me);
    }
  }
}

inline int ppo_grid(int64_t n, int threads, int unroll, bool vec, int cus, int per_cu) {
  const int64_t per_block = (int64_t)threads * unroll * (vec ? 4 : 1);
  int64_t blocks = (n + per_block - 1) / per_block;
  const int64_t cap = (int64_t)cus * per_cu;
  if (blocks > cap) blocks = cap;
  if (blocks > PpoWorkspace::kMaxBlocks) blocks = PpoWorkspace::kMaxBlocks;
  return blocks < 1 ? 1 : (int)blocks;
}

}  // namespace taskops
