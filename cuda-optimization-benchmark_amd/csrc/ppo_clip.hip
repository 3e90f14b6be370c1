// ppo_clip on gfx950: PPO clipped objective and its five diagnostics in one pass.
//
// Op: tasks/ppo_clip/reference.py:27-39 (fp64 oracle :42-45, eps rounded to fp32 first);
// drop-in signature tasks/ppo_clip/tests/task.json:3, replacing
// reference/ppo_clip/solution.cu:165-182.  The entropy variant adds TorchRL
// ClipPPOLoss's entropy bonus (mean entropy and -coef * mean entropy).
//
// HBM-bound: 12 bytes per sample (16 with entropy).  Per sample, with lw = cur - old:
//   r = exp(lw); gain = A * (A > 0 && lw > log1p(eps) ? 1 + eps
//                         : A < 0 && lw < log1p(-eps) ? 1 - eps : r)
// which equals min(r*A, exp(clamp(lw, log1p(-eps), log1p(eps)))*A); the clip test runs on
// the exact fp64 difference against the fp64 bounds, so the clip count matches the fp64
// reference.  ESS uses exp(2 lse(lw) - lse(2 lw)) / N = (sum r)^2 / (N sum r^2).
// Per-thread sums are fp32 over one unrolled iteration, then fp64; the finishing
// workgroup combines the per-workgroup records in a fixed order.
#include "common.hpp"

namespace taskops {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 2;
constexpr int kMaxBlocks = 4096;
constexpr int kBlocksPerCU = 8;
constexpr int kFields = 7;  // gain, clipped, kl, sum r, sum r^2, sum entropy, max r

struct PpoWorkspace {
  double partial[kMaxBlocks][8];
  unsigned ticket;
};

using f32x4 = float __attribute__((ext_vector_type(4)));

struct Acc {
  float gain = 0.f, kl = 0.f, sr = 0.f, sr2 = 0.f, se = 0.f, maxr = 0.f;
  unsigned clipped = 0;
};

struct Params {
  double lo, hi;     // log1p(-eps), log1p(eps) in fp64
  float lo_ratio;    // 1 - eps
  float hi_ratio;    // 1 + eps
};

__device__ __forceinline__ void sample(Acc& s, float cur, float old, float adv, const Params& p) {
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

template <bool kVec, bool kEntropy>
__global__ __launch_bounds__(kThreads) void ppo_clip_kernel(
    int64_t n, const float* __restrict__ cur, const float* __restrict__ old,
    const float* __restrict__ adv, const float* __restrict__ ent, Params p, float coef,
    PpoWorkspace* __restrict__ ws, float* __restrict__ out) {
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
        c[u] = c4[i + u * stride];
        o[u] = o4[i + u * stride];
        a[u] = a4[i + u * stride];
        if constexpr (kEntropy) e[u] = e4[i + u * stride];
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
      const f32x4 c = c4[i], o = o4[i], a = a4[i];
      sample(s, c.x, o.x, a.x, p);
      sample(s, c.y, o.y, a.y, p);
      sample(s, c.z, o.z, a.z, p);
      sample(s, c.w, o.w, a.w, p);
      if constexpr (kEntropy) {
        const f32x4 e = e4[i];
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
  if (threadIdx.x < kFields) {
    const int f = threadIdx.x;
    double t = lds[f][0];
    for (int w = 1; w < kThreads / kWave; ++w)
      t = (f == kFields - 1) ? fmax(t, lds[f][w]) : t + lds[f][w];
    ws->partial[blockIdx.x][f] = t;
  }
  if (!arrive_is_last(&ws->ticket, &last)) return;

  // Finishing workgroup: wave w reduces fields w and w + 4 over all workgroup records
  // (ratios are positive, so 0 is the identity of the max as well as of the sums).
  for (int f = wave; f < kFields; f += kThreads / kWave) {
    double t = 0.0;
    for (int j = lane; j < (int)gridDim.x; j += kWave) {
      const double x = load_coherent(&ws->partial[j][f]);
      t = (f == kFields - 1) ? fmax(t, x) : t + x;
    }
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
    reset_ticket(&ws->ticket);
  }
}

template <bool kEntropy>
hipError_t launch(int32_t B, int32_t T, int32_t H, const float* cur, const float* old,
                  const float* adv, const float* ent, float eps, float coef, float* out,
                  hipStream_t stream) {
  const int64_t n = (int64_t)B * T * H;
  if (B <= 0 || T <= 0 || H <= 0) return hipErrorInvalidValue;
  void* wsp = nullptr;
  hipError_t e = workspace(kSlotPpo, sizeof(PpoWorkspace), stream, &wsp);
  if (e != hipSuccess) return e;
  auto* ws = static_cast<PpoWorkspace*>(wsp);
  Params p;
  p.lo = log1p(-(double)eps);
  p.hi = log1p((double)eps);
  p.lo_ratio = (float)(1.0 - (double)eps);
  p.hi_ratio = (float)(1.0 + (double)eps);
  uintptr_t bits = reinterpret_cast<uintptr_t>(cur) | reinterpret_cast<uintptr_t>(old) |
                   reinterpret_cast<uintptr_t>(adv);
  if (kEntropy) bits |= reinterpret_cast<uintptr_t>(ent);
  const bool vec = (bits & 15) == 0;
  const int64_t per_block = (int64_t)kThreads * kUnroll * (vec ? 4 : 1);
  int64_t blocks = (n + per_block - 1) / per_block;
  const int64_t cap = (int64_t)device_cu_count() * kBlocksPerCU;
  if (blocks > cap) blocks = cap;
  if (blocks > kMaxBlocks) blocks = kMaxBlocks;
  if (blocks < 1) blocks = 1;
  if (vec)
    hipLaunchKernelGGL((ppo_clip_kernel<true, kEntropy>), dim3((unsigned)blocks), dim3(kThreads),
                       0, stream, n, cur, old, adv, ent, p, coef, ws, out);
  else
    hipLaunchKernelGGL((ppo_clip_kernel<false, kEntropy>), dim3((unsigned)blocks), dim3(kThreads),
                       0, stream, n, cur, old, adv, ent, p, coef, ws, out);
  return hipGetLastError();
}

}  // namespace
}  // namespace taskops

extern "C" hipError_t taskops_ppo_clip(int32_t B, int32_t T, int32_t H,
                                       const float* current_log_prob, const float* old_log_prob,
                                       const float* advantage, float clip_epsilon, float* output,
                                       hipStream_t stream) {
  return taskops::launch<false>(B, T, H, current_log_prob, old_log_prob, advantage, nullptr,
                                clip_epsilon, 0.0f, output, stream);
}

extern "C" hipError_t taskops_ppo_clip_entropy(int32_t B, int32_t T, int32_t H,
                                               const float* current_log_prob,
                                               const float* old_log_prob, const float* advantage,
                                               const float* entropy, float clip_epsilon,
                                               float entropy_coef, float* output,
                                               hipStream_t stream) {
  return taskops::launch<true>(B, T, H, current_log_prob, old_log_prob, advantage, entropy,
                               clip_epsilon, entropy_coef, output, stream);
}
