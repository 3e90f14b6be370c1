// quantize_e4m3 on gfx950: per-tensor max-abs OCP e4m3 quantisation, the step that
// produces fp8_linear's operands.
//
// Op: tasks/fp8_linear/reference.py:15-18 (`_quantize`):
//   scale = fp32(448 / max(max|x|, 1e-9))      quotient in fp64 (a Python float), one rounding
//   q     = e4m3(clamp(x * scale, -448, 448))   fp32 product, round-to-nearest-even cast
// A NaN in x makes amax, scale and every q NaN: torch's max, Python's max(nan, 1e-9) and
// the casts all keep it.
//
// HBM-bound; algorithmic bytes are 4 in + 1 out per element.  The max is taken over |x|
// as raw bits: for |x| the IEEE order is the unsigned-integer order and every NaN sorts
// above inf, so an integer max propagates NaN.  Conversion is v_cvt_pk_fp8_f32.
//
// Two launches (unaligned operands, or more chunks than can be resident at once): qz_amax
// writes one partial max per workgroup; qz_cast reduces those partials (a few KiB from L2),
// derives the scale and converts, reading x a second time.
//
// The kernels walk x in chunks of 16384 elements per 512-thread workgroup and step.  A
// thread issues all 8 of its 16-byte loads of a chunk before it uses any (32 floats in
// registers), so each wave keeps 8 KiB in flight: at one chunk per workgroup, which a
// 4096 x 4096 operand is on 256 CUs, a kernel is one round trip of loads.  Element
// base + 4 * (k * 512 + t) + c of a chunk belongs to thread t, so every load and store
// instruction of a wave covers contiguous memory.  The same chunk as 256 threads x 16
// loads was 17.83-17.84 us per fused call against 17.58-17.61 (A/B on two boxes, same
// bits); 512 x 16 and 1024 x 8 were in between, 1024 x 16 slower (22.4).
//
// One launch (qz_fused, when the grid fits the resident capacity): each workgroup keeps its
// chunk in registers, the workgroups combine their maxima through a grid barrier, and each
// converts the chunk it holds, so x is read once.  The barrier is a plain launch sized by
// the occupancy API (a cooperative launch, which guarantees residency, costs about 100 us
// per launch on this stack).  Residency is not guaranteed (another stream's kernels can
// hold CUs), so the wait is bounded: a workgroup that times out reads all of x for the max
// itself.  The max is exact and order-free, so both paths give identical bits, every wave
// exits, and no result depends on the timing.
#include "common.hpp"

namespace taskops {
namespace {

constexpr int kThreads = 512;
constexpr int kVecs = 8;                                        // f32x4 per thread per chunk
constexpr int64_t kChunk = (int64_t)kThreads * kVecs * 4;        // elements per chunk
constexpr int kPerThread = 16;  // elements per thread per step of the unaligned kernels
constexpr int kMaxPartials = 2048;
using f32x4 = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned abs_bits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

__device__ __forceinline__ unsigned wave_max_u32(unsigned v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, (unsigned)__shfl_xor((int)v, off, kWave));
  return v;
}

// Max over the workgroup; valid in every thread.
__device__ __forceinline__ unsigned block_max_u32(unsigned v, unsigned* lds) {
  v = wave_max_u32(v);
  if (threadIdx.x % kWave == 0) lds[threadIdx.x / kWave] = v;
  __syncthreads();
  unsigned m = 0u;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) m = max(m, lds[w]);
  __syncthreads();
  return m;
}

// This thread's 64 elements of the chunk at `base` (x 16-byte aligned); elements at or
// beyond n read as 0, which never raises the max.
__device__ __forceinline__ void load_chunk(const float* __restrict__ x, int64_t n, int64_t base, f32x4 (&v)[kVecs]) {
  if (base + kChunk <= n) {
    const f32x4* p = reinterpret_cast<const f32x4*>(x + base) + threadIdx.x;
#pragma unroll
    for (int k = 0; k < kVecs; ++k) v[k] = __builtin_nontemporal_load(p + k * kThreads);
    return;
  }
#pragma unroll
  for (int k = 0; k < kVecs; ++k) {
    const int64_t i = base + 4 * ((int64_t)k * kThreads + threadIdx.x);
    if (i + 4 <= n) {
      v[k] = *reinterpret_cast<const f32x4*>(x + i);
    } else {
      v[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (i < n) v[k].x = x[i];
      if (i + 1 < n) v[k].y = x[i + 1];
      if (i + 2 < n) v[k].z = x[i + 2];
    }
  }
}

__device__ __forceinline__ unsigned chunk_max(const f32x4 (&v)[kVecs], unsigned m) {
#pragma unroll
  for (int k = 0; k < kVecs; ++k)
    m = max(max(m, max(abs_bits(v[k].x), abs_bits(v[k].y))), max(abs_bits(v[k].z), abs_bits(v[k].w)));
  return m;
}

// Two fp32 values to e4m3 bytes (round to nearest even) in bytes 0-1 (kHi false) or 2-3
// of `word`, the other half kept; the inputs are already within [-448, 448] or NaN.
template <bool kHi>
__device__ __forceinline__ unsigned cvt2(float a, float b, unsigned word) {
  return (unsigned)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)word, kHi);
}

// clamp(v * scale, -448, 448) with NaN kept (torch.clamp leaves NaN).
__device__ __forceinline__ float scaled(float v, float scale) {
  const float s = v * scale;
  return s < -448.0f ? -448.0f : (s > 448.0f ? 448.0f : s);
}

// Four fp32 values, scaled and clamped, to e4m3 codes packed in one 32-bit word.
__device__ __forceinline__ unsigned cvt4(f32x4 v, float scale) {
  const unsigned w = cvt2<false>(scaled(v.x, scale), scaled(v.y, scale), 0u);
  return cvt2<true>(scaled(v.z, scale), scaled(v.w, scale), w);
}

// fp32 scale from the max bits: Python's max(amax, 1e-9) keeps a NaN amax; 448 / it is
// evaluated in fp64 and rounded once to fp32.
__device__ __forceinline__ float scale_from(unsigned m) {
  const float amax = __uint_as_float(m);
  const double den = (m > 0x7F800000u) ? (double)amax : fmax((double)amax, 1e-9);
  return (float)(448.0 / den);
}

// Codes of this thread's part of the chunk at `base` (q 4-byte aligned).  A whole chunk's
// stores are non-temporal (each instruction writes 256 contiguous bytes, whole lines), so
// the codes do not sit dirty in the L2s for the end of the kernel to write back: 19.5-19.6
// -> 17.6-17.7 us per call at 4096 x 4096 (A/B on one box, both orders, same bits).
__device__ __forceinline__ void store_chunk(uint8_t* __restrict__ q, int64_t n, int64_t base,
                                            const f32x4 (&v)[kVecs], float scale) {
  if (base + kChunk <= n) {
    unsigned* out = reinterpret_cast<unsigned*>(q + base) + threadIdx.x;
#pragma unroll
    for (int k = 0; k < kVecs; ++k) __builtin_nontemporal_store(cvt4(v[k], scale), out + k * kThreads);
    return;
  }
#pragma unroll
  for (int k = 0; k < kVecs; ++k) {
    const int64_t i = base + 4 * ((int64_t)k * kThreads + threadIdx.x);
    const unsigned w = cvt4(v[k], scale);
    if (i + 4 <= n) {
      *reinterpret_cast<unsigned*>(q + i) = w;
    } else {
      for (int c = 0; c < 3; ++c)
        if (i + c < n) q[i + c] = (uint8_t)(w >> (8 * c));
    }
  }
}

// ---------------------------------------------------------------------------------------
// Aligned kernels: x 16-byte aligned (and q 4-byte aligned for the cast).
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void qz_amax(const float* __restrict__ x, int64_t n,
                                                    unsigned* __restrict__ partial) {
  __shared__ unsigned lds[kThreads / kWave];
  unsigned m = 0u;
  for (int64_t base = (int64_t)blockIdx.x * kChunk; base < n; base += (int64_t)gridDim.x * kChunk) {
    f32x4 v[kVecs];
    load_chunk(x, n, base, v);
    m = chunk_max(v, m);
  }
  m = block_max_u32(m, lds);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

__global__ __launch_bounds__(kThreads) void qz_cast(const float* __restrict__ x, int64_t n,
                                                    const unsigned* __restrict__ partial, int nparts,
                                                    uint8_t* __restrict__ q, float* __restrict__ scale_out) {
  __shared__ unsigned lds[kThreads / kWave];
  int64_t base = (int64_t)blockIdx.x * kChunk;
  // The first chunk's loads go out before the partials are read, so the two overlap.
  f32x4 v[kVecs];
  if (base < n) load_chunk(x, n, base, v);
  unsigned m = 0u;
  for (int i = threadIdx.x; i < nparts; i += kThreads) m = max(m, partial[i]);
  m = block_max_u32(m, lds);
  const float scale = scale_from(m);
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
  if (base >= n) return;
  store_chunk(q, n, base, v, scale);
  for (base += (int64_t)gridDim.x * kChunk; base < n; base += (int64_t)gridDim.x * kChunk) {
    load_chunk(x, n, base, v);
    store_chunk(q, n, base, v, scale);
  }
}

// ---------------------------------------------------------------------------------------
// Unaligned kernels (element loads and byte stores), for any x and q.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void qz_amax_any(const float* __restrict__ x, int64_t n,
                                                        unsigned* __restrict__ partial) {
  __shared__ unsigned lds[kThreads / kWave];
  unsigned m = 0u;
  const int64_t stride = (int64_t)gridDim.x * kThreads * kPerThread;
  for (int64_t i0 = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * kPerThread; i0 < n; i0 += stride)
    for (int64_t i = i0; i < i0 + kPerThread && i < n; ++i) m = max(m, abs_bits(x[i]));
  m = block_max_u32(m, lds);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

__global__ __launch_bounds__(kThreads) void qz_cast_any(const float* __restrict__ x, int64_t n,
                                                        const unsigned* __restrict__ partial, int nparts,
                                                        uint8_t* __restrict__ q, float* __restrict__ scale_out) {
  __shared__ unsigned lds[kThreads / kWave];
  unsigned m = 0u;
  for (int i = threadIdx.x; i < nparts; i += kThreads) m = max(m, partial[i]);
  m = block_max_u32(m, lds);
  const float scale = scale_from(m);
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
  const int64_t stride = (int64_t)gridDim.x * kThreads * kPerThread;
  for (int64_t i0 = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * kPerThread; i0 < n; i0 += stride)
    for (int64_t i = i0; i < i0 + kPerThread && i < n; ++i)
      q[i] = (uint8_t)(cvt2<false>(scaled(x[i], scale), 0.0f, 0u) & 0xFFu);
}

// ---------------------------------------------------------------------------------------
// Fused single pass.
// ---------------------------------------------------------------------------------------
// Barrier words in the workspace after the partials, one per 64-byte line, in two sets;
// the parity word says which set a launch uses.  Set s holds group g's arrival count and
// max and the top arrival count.  RMWs on one address serialise at the coherence point
// (about 12 ns each), so arrival is two-level: workgroup b folds its max into group b % 16's
// max and then counts itself in the group (each RMW's result is used before the next is
// issued, which orders them at the coherence point); a group's last arrival counts the group
// in at the top.  The grid's last arrival clears the other set (the previous launch's, which
// the next launch uses) and flips the parity.  Waiters poll the parity word, which no RMW
// touches, until it differs from what they read at start, then read the group maxima, final
// by then, and take their max: from the last arrival's data that is two RMWs, the group's
// top RMW, the flip, one poll and one read.  A set is only cleared by the launch after the
// one that reads it, every launch leaves the next one a cleared set, no host reset is needed
// and a captured graph replays correctly.
constexpr int kQzGroups = 16;
constexpr int kQzLine = 16;  // unsigned per 64-byte line
enum QzWord : int { kQzGroupCount = 0, kQzGroupMax = kQzGroups, kQzTopCount = 2 * kQzGroups, kQzSetWords };
constexpr int kQzParity = 2 * kQzSetWords;  // after both sets
constexpr int kQzWords = kQzParity + 1;
static_assert(kQzSetWords <= kWave, "the grid's last arrival clears a set with one store per lane of a wave");
constexpr unsigned kQzSpinDefault = 1u << 14;  // polls of the parity (~0.5-1 us each) before the fallback

__device__ __forceinline__ unsigned* qz_word(unsigned* bar, unsigned set, int w, int i = 0) {
  return bar + ((int)set * kQzSetWords + w + i) * kQzLine;
}
__device__ __forceinline__ unsigned* qz_parity(unsigned* bar) { return bar + kQzParity * kQzLine; }
__device__ __forceinline__ unsigned qz_load(unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void qz_store(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned qz_max(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned qz_add(unsigned* p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Requires x 16-byte and q 4-byte aligned and gridDim.x = ceil(n / kChunk).  Thread 0 of
// each workgroup runs the barrier; every RMW's returned value is used before the next
// one is issued, which orders them at the coherence point.  8 waves per SIMD (at most 64
// VGPRs) make 4 workgroups per CU resident, 1024 on 256 CUs: a 4096 x 4096 operand's chunks.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8))) void qz_fused(
    const float* __restrict__ x, int64_t n, uint8_t* __restrict__ q, float* __restrict__ scale_out,
    unsigned* __restrict__ bar, unsigned spin_limit) {
  __shared__ unsigned lds[kThreads / kWave];
  __shared__ unsigned gmax_s, fallback_s;
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  f32x4 v[kVecs];
  load_chunk(x, n, base, v);
  // The parity is read behind the chunk's loads; it only has to be read before this
  // workgroup arrives.
  unsigned parity = 0u;
  if (threadIdx.x == 0) parity = qz_load(qz_parity(bar));
  const unsigned m = block_max_u32(chunk_max(v, 0u), lds);

  if (threadIdx.x < kWave) {  // wave 0 runs the barrier; lane 0 makes the RMWs
    const int lane = threadIdx.x;
    parity = (unsigned)__shfl((int)parity, 0, kWave);
    const unsigned set = parity & 1u;
    const unsigned grid = gridDim.x, g = blockIdx.x % kQzGroups;
    const unsigned groups = grid < kQzGroups ? grid : kQzGroups;
    const unsigned members = grid / kQzGroups + (g < grid % kQzGroups ? 1u : 0u);
    bool last = false;
    if (lane == 0) {
      const unsigned r = qz_max(qz_word(bar, set, kQzGroupMax, g), m);
      asm volatile("" ::"v"(r));
      if (qz_add(qz_word(bar, set, kQzGroupCount, g)) == members - 1)  // the group's last arrival
        last = qz_add(qz_word(bar, set, kQzTopCount)) == groups - 1;     // the grid's last arrival
    }
    if (__builtin_amdgcn_ballot_w64(last) != 0ull) {
      if (lane < kQzSetWords) qz_store(qz_word(bar, set ^ 1u, 0, lane), 0u);
      if (lane == 0) qz_store(qz_parity(bar), parity ^ 1u);
    }
    bool done = false;
    if (lane == 0) {
      for (unsigned i = 0; i < spin_limit; ++i) {
        if (qz_load(qz_parity(bar)) != parity) {
          done = true;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    done = __builtin_amdgcn_ballot_w64(done) != 0ull;
    unsigned gm = 0u;
    if (done) gm = wave_max_u32((unsigned)lane < groups ? qz_load(qz_word(bar, set, kQzGroupMax, lane)) : 0u);
    if (lane == 0) {
      fallback_s = done ? 0u : 1u;
      gmax_s = gm;
    }
  }
  __syncthreads();
  unsigned gm = gmax_s;
  if (fallback_s) {  // the barrier did not complete in time: this workgroup finds the max itself
    unsigned mm = 0u;    // (one 16-byte load at a time: the chunk in v stays in registers)
    const int64_t n4 = n & ~(int64_t)3;
    for (int64_t i = 4 * (int64_t)threadIdx.x; i < n4; i += 4 * kThreads) {
      const f32x4 w = *reinterpret_cast<const f32x4*>(x + i);
      mm = max(max(mm, max(abs_bits(w.x), abs_bits(w.y))), max(abs_bits(w.z), abs_bits(w.w)));
    }
    if ((int64_t)threadIdx.x < n - n4) mm = max(mm, abs_bits(x[n4 + threadIdx.x]));
    gm = block_max_u32(mm, lds);
  }
  const float scale = scale_from(gm);
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
  store_chunk(q, n, base, v, scale);
}

unsigned g_qz_spin_limit = kQzSpinDefault;
int g_qz_capacity[64];  // resident qz_fused workgroups per device (0: not yet known, -1: none)

int fused_capacity() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int cap = __atomic_load_n(&g_qz_capacity[dev], __ATOMIC_RELAXED);
  if (cap != 0) return cap > 0 ? cap : 0;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(qz_fused), kThreads, 0) !=
          hipSuccess ||
      per_cu <= 0) {
    (void)hipGetLastError();
    cap = -1;
  } else {
    cap = per_cu * device_cu_count();
  }
  __atomic_store_n(&g_qz_capacity[dev], cap, __ATOMIC_RELAXED);
  return cap > 0 ? cap : 0;
}

// Workgroups for n elements at `per_block` elements per step: enough for one step each,
// at most `per_cu` per CU and kMaxPartials.
int grid_for(int64_t n, int64_t per_block, int per_cu) {
  int64_t g = (n + per_block - 1) / per_block;
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  if (g > cap) g = cap;
  if (g > kMaxPartials) g = kMaxPartials;
  return (int)(g < 1 ? 1 : g);
}

}  // namespace
}  // namespace taskops

using namespace taskops;

extern "C" hipError_t taskops_quantize_e4m3(const float* x, int64_t n, uint8_t* q, float* scale,
                                            hipStream_t stream) {
  if (n < 0) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;  // nothing to quantise; *scale is left as it is
  void* wsp = nullptr;
  hipError_t e = workspace(kSlotQuant, (kMaxPartials + kQzWords * kQzLine) * sizeof(unsigned), stream, &wsp);
  if (e != hipSuccess) return e;
  auto* partial = static_cast<unsigned*>(wsp);
  const bool vx = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  const bool vq = (reinterpret_cast<uintptr_t>(q) & 3) == 0;
  const int64_t chunks = (n + kChunk - 1) / kChunk;
  if (vx && vq && chunks <= fused_capacity()) {
    hipLaunchKernelGGL(qz_fused, dim3((unsigned)chunks), dim3(kThreads), 0, stream, x, n, q, scale,
                       partial + kMaxPartials, g_qz_spin_limit);
    return hipGetLastError();
  }
  if (vx && vq) {
    // Up to 4 workgroups of 8 waves per CU (qz_amax holds 42 VGPRs, qz_cast 72, which
    // leaves room for 3); 1024 workgroups cover 4096 x 4096 in one chunk each.
    const int g = grid_for(n, kChunk, 4);
    hipLaunchKernelGGL(qz_amax, dim3(g), dim3(kThreads), 0, stream, x, n, partial);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(qz_cast, dim3(g), dim3(kThreads), 0, stream, x, n, partial, g, q, scale);
    return hipGetLastError();
  }
  // 2 and 4 workgroups of 8 waves per CU: 16 and 32 waves.
  const int g1 = grid_for(n, (int64_t)kThreads * kPerThread, 2);
  hipLaunchKernelGGL(qz_amax_any, dim3(g1), dim3(kThreads), 0, stream, x, n, partial);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int g2 = grid_for(n, (int64_t)kThreads * kPerThread, 4);
  hipLaunchKernelGGL(qz_cast_any, dim3(g2), dim3(kThreads), 0, stream, x, n, partial, g1, q, scale);
  return hipGetLastError();
}

// Test hook: the polls of the fused kernel's bounded wait before a workgroup falls back to
// finding the max itself (0 sends every workgroup to the fallback).  Not thread-safe; for
// tests that check both paths give the same bits.
extern "C" void taskops_testing_quantize_spin_limit(unsigned polls) { g_qz_spin_limit = polls; }
