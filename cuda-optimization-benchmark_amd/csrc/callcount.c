/* HIP API call counter (libhipcount.so): measures what one libtaskops call asks of the HIP
 * runtime — allocations, host copies, synchronisations, launches, and work put on any
 * stream other than the caller's.
 *
 * Counterpart of graders/interpose.c:14-115, which the reference preloads into its driver
 * and arms around the graded call (graders/child.py:103-118).  Here the library is loaded
 * with RTLD_GLOBAL before the process loads the HIP runtime, so its definitions of the
 * hooked hip* functions precede the runtime's in the global lookup scope and every later
 * caller (libtaskops, torch) binds to them.  Nothing is preloaded through the environment.
 * The library does not link the HIP runtime: each hook resolves the runtime's own function
 * on first use (the next definition after this library, else the already-loaded
 * libamdhip64 by soname) and forwards to it unchanged.
 *
 * Counting happens only while armed.  A hooked call made by the runtime from inside
 * another hooked call (on the same thread) is not counted again.
 *
 * Built by build.py with gcc (host code only): lib/libhipcount.so.
 */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <stddef.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

/* Categories, in the order hipcount_read() reports them. */
enum {
  CC_ALLOC,        /* device, host or managed allocation or free */
  CC_HOST_COPY,    /* copy with a host source or destination */
  CC_DEVICE_SYNC,  /* hipDeviceSynchronize, or a sync of the null/legacy stream */
  CC_OTHER_STREAM, /* launch, copy or memset on a stream other than the caller's */
  CC_STREAM_SYNC,  /* hipStreamSynchronize of a created stream */
  CC_LAUNCH,       /* kernel or graph launch, any stream */
  CC_MEMSET,       /* memset, any stream */
  CC_DEVICE_COPY,  /* device-to-device copy, any stream */
  CC_N
};
static const char kNames[] =
    "alloc,host_copy,device_sync,other_stream,stream_sync,launch,memset,device_copy";

static long g_counts[CC_N];
static int g_armed;
static hipStream_t g_stream; /* the stream the measured call was given */
static __thread int t_depth;

/* ---- control API (called through ctypes) ---- */
void hipcount_arm(int on) { __atomic_store_n(&g_armed, on ? 1 : 0, __ATOMIC_SEQ_CST); }
void hipcount_reset(void) {
  for (int i = 0; i < CC_N; ++i) __atomic_store_n(&g_counts[i], 0, __ATOMIC_SEQ_CST);
}
void hipcount_set_stream(hipStream_t s) { g_stream = s; }
int hipcount_read(long* out, int n) {
  for (int i = 0; i < n && i < CC_N; ++i) out[i] = __atomic_load_n(&g_counts[i], __ATOMIC_SEQ_CST);
  return CC_N;
}
const char* hipcount_names(void) { return kNames; }

/* ---- helpers ---- */
static void note(int c) {
  if (t_depth == 0 && __atomic_load_n(&g_armed, __ATOMIC_RELAXED)) __atomic_fetch_add(&g_counts[c], 1, __ATOMIC_RELAXED);
}
static void note_on(int c, hipStream_t s) {
  note(c);
  if (s != g_stream) note(CC_OTHER_STREAM);
}

static void* resolve(const char* name) {
  void* f = dlsym(RTLD_NEXT, name);
  if (!f) {
    static const char* const sonames[] = {"libamdhip64.so.7", "libamdhip64.so"};
    for (size_t i = 0; !f && i < sizeof sonames / sizeof *sonames; ++i) {
      void* h = dlopen(sonames[i], RTLD_LAZY | RTLD_NOLOAD);
      if (h) f = dlsym(h, name);
    }
  }
  return f;
}

/* Declares `real` as the runtime's `name`, resolved once; returns an error if absent. */
#define RESOLVE(name)                                                    \
  static __typeof__(&name) real;                                         \
  if (!real) real = (__typeof__(&name))resolve(#name);                   \
  if (!real) return hipErrorSharedObjectSymbolNotFound

/* Calls the runtime with nested hooks muted. */
#define FORWARD(...)                \
  do {                              \
    ++t_depth;                      \
    hipError_t e_ = real(__VA_ARGS__); \
    --t_depth;                      \
    return e_;                      \
  } while (0)

/* ---- where the two ends of a copy live ----
 * A copy is a host copy when either end is host memory.  An explicit kind names both ends;
 * hipMemcpyDefault (and any kind this file does not know) asks the runtime about each
 * pointer, and memory the runtime does not know counts as host memory. */
enum copy_end { END_HOST, END_DEVICE };

static enum copy_end locate(const void* p) {
  static __typeof__(&hipPointerGetAttributes) attrs;
  if (!attrs) attrs = (__typeof__(&hipPointerGetAttributes))resolve("hipPointerGetAttributes");
  if (!attrs) return END_HOST;
  hipPointerAttribute_t a;
  memset(&a, 0, sizeof a);
  ++t_depth;
  const hipError_t e = attrs(&a, p);
  --t_depth;
  if (e != hipSuccess) return END_HOST;
  return (a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged) ? END_DEVICE : END_HOST;
}

/* Ends of a copy from `src` to `dst`; a NULL pointer is an end known to be device memory
 * (a symbol), located only when the kind does not say. */
static void copy_ends(hipMemcpyKind k, const void* dst, const void* src, enum copy_end* from,
                      enum copy_end* to) {
  switch (k) {
    case hipMemcpyHostToHost: *from = END_HOST; *to = END_HOST; return;
    case hipMemcpyHostToDevice: *from = END_HOST; *to = END_DEVICE; return;
    case hipMemcpyDeviceToHost: *from = END_DEVICE; *to = END_HOST; return;
    case hipMemcpyDeviceToDevice:
    case hipMemcpyDeviceToDeviceNoCU: *from = END_DEVICE; *to = END_DEVICE; return;
    default:
      *from = src ? locate(src) : END_DEVICE;
      *to = dst ? locate(dst) : END_DEVICE;
      return;
  }
}

/* A copy on stream s (synchronous copies run on the null stream). */
static void note_copy(hipMemcpyKind k, const void* dst, const void* src, hipStream_t s) {
  enum copy_end from, to;
  copy_ends(k, dst, src, &from, &to);
  if (from == END_HOST || to == END_HOST)
    note(CC_HOST_COPY);
  else
    note_on(CC_DEVICE_COPY, s);
}

/* ---- allocation (hipMallocHost is deprecated in the headers but still exported) ---- */
hipError_t hipMalloc(void** p, size_t n) { RESOLVE(hipMalloc); note(CC_ALLOC); FORWARD(p, n); }
hipError_t hipMallocManaged(void** p, size_t n, unsigned f) { RESOLVE(hipMallocManaged); note(CC_ALLOC); FORWARD(p, n, f); }
hipError_t hipHostMalloc(void** p, size_t n, unsigned f) { RESOLVE(hipHostMalloc); note(CC_ALLOC); FORWARD(p, n, f); }
hipError_t hipHostAlloc(void** p, size_t n, unsigned f) { RESOLVE(hipHostAlloc); note(CC_ALLOC); FORWARD(p, n, f); }
hipError_t hipMallocHost(void** p, size_t n) { RESOLVE(hipMallocHost); note(CC_ALLOC); FORWARD(p, n); }
hipError_t hipMallocPitch(void** p, size_t* pitch, size_t w, size_t h) { RESOLVE(hipMallocPitch); note(CC_ALLOC); FORWARD(p, pitch, w, h); }
hipError_t hipMallocAsync(void** p, size_t n, hipStream_t s) { RESOLVE(hipMallocAsync); note(CC_ALLOC); FORWARD(p, n, s); }
hipError_t hipMallocFromPoolAsync(void** p, size_t n, hipMemPool_t pool, hipStream_t s) {
  RESOLVE(hipMallocFromPoolAsync); note(CC_ALLOC); FORWARD(p, n, pool, s);
}
hipError_t hipExtMallocWithFlags(void** p, size_t n, unsigned f) { RESOLVE(hipExtMallocWithFlags); note(CC_ALLOC); FORWARD(p, n, f); }
hipError_t hipFree(void* p) { RESOLVE(hipFree); note(CC_ALLOC); FORWARD(p); }
hipError_t hipHostFree(void* p) { RESOLVE(hipHostFree); note(CC_ALLOC); FORWARD(p); }
hipError_t hipFreeHost(void* p) { RESOLVE(hipFreeHost); note(CC_ALLOC); FORWARD(p); }
hipError_t hipFreeAsync(void* p, hipStream_t s) { RESOLVE(hipFreeAsync); note(CC_ALLOC); FORWARD(p, s); }

/* ---- copies ---- */
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind k) {
  RESOLVE(hipMemcpy); note_copy(k, d, s, NULL); FORWARD(d, s, n, k);
}
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t st) {
  RESOLVE(hipMemcpyAsync); note_copy(k, d, s, st); FORWARD(d, s, n, k, st);
}
hipError_t hipMemcpyWithStream(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t st) {
  RESOLVE(hipMemcpyWithStream); note_copy(k, d, s, st); FORWARD(d, s, n, k, st);
}
hipError_t hipMemcpyHtoD(hipDeviceptr_t d, const void* s, size_t n) { RESOLVE(hipMemcpyHtoD); note(CC_HOST_COPY); FORWARD(d, s, n); }
hipError_t hipMemcpyDtoH(void* d, hipDeviceptr_t s, size_t n) { RESOLVE(hipMemcpyDtoH); note(CC_HOST_COPY); FORWARD(d, s, n); }
hipError_t hipMemcpyDtoD(hipDeviceptr_t d, hipDeviceptr_t s, size_t n) {
  RESOLVE(hipMemcpyDtoD); note_on(CC_DEVICE_COPY, NULL); FORWARD(d, s, n);
}
hipError_t hipMemcpyHtoDAsync(hipDeviceptr_t d, const void* s, size_t n, hipStream_t st) {
  RESOLVE(hipMemcpyHtoDAsync); note(CC_HOST_COPY); FORWARD(d, s, n, st);
}
hipError_t hipMemcpyDtoHAsync(void* d, hipDeviceptr_t s, size_t n, hipStream_t st) {
  RESOLVE(hipMemcpyDtoHAsync); note(CC_HOST_COPY); FORWARD(d, s, n, st);
}
hipError_t hipMemcpyDtoDAsync(hipDeviceptr_t d, hipDeviceptr_t s, size_t n, hipStream_t st) {
  RESOLVE(hipMemcpyDtoDAsync); note_on(CC_DEVICE_COPY, st); FORWARD(d, s, n, st);
}
hipError_t hipMemcpy2D(void* d, size_t dp, const void* s, size_t sp, size_t w, size_t h, hipMemcpyKind k) {
  RESOLVE(hipMemcpy2D); note_copy(k, d, s, NULL); FORWARD(d, dp, s, sp, w, h, k);
}
hipError_t hipMemcpy2DAsync(void* d, size_t dp, const void* s, size_t sp, size_t w, size_t h, hipMemcpyKind k,
                            hipStream_t st) {
  RESOLVE(hipMemcpy2DAsync); note_copy(k, d, s, st); FORWARD(d, dp, s, sp, w, h, k, st);
}
/* Symbol copies: the symbol end is device memory (passed as NULL to note_copy). */
hipError_t hipMemcpyToSymbol(const void* sym, const void* s, size_t n, size_t off, hipMemcpyKind k) {
  RESOLVE(hipMemcpyToSymbol); note_copy(k, NULL, s, NULL); FORWARD(sym, s, n, off, k);
}
hipError_t hipMemcpyToSymbolAsync(const void* sym, const void* s, size_t n, size_t off, hipMemcpyKind k,
                                  hipStream_t st) {
  RESOLVE(hipMemcpyToSymbolAsync); note_copy(k, NULL, s, st); FORWARD(sym, s, n, off, k, st);
}
hipError_t hipMemcpyFromSymbol(void* d, const void* sym, size_t n, size_t off, hipMemcpyKind k) {
  RESOLVE(hipMemcpyFromSymbol); note_copy(k, d, NULL, NULL); FORWARD(d, sym, n, off, k);
}
hipError_t hipMemcpyFromSymbolAsync(void* d, const void* sym, size_t n, size_t off, hipMemcpyKind k,
                                    hipStream_t st) {
  RESOLVE(hipMemcpyFromSymbolAsync); note_copy(k, d, NULL, st); FORWARD(d, sym, n, off, k, st);
}

/* ---- memsets (synchronous ones run on the null stream) ---- */
hipError_t hipMemset(void* d, int v, size_t n) { RESOLVE(hipMemset); note_on(CC_MEMSET, NULL); FORWARD(d, v, n); }
hipError_t hipMemsetAsync(void* d, int v, size_t n, hipStream_t st) {
  RESOLVE(hipMemsetAsync); note_on(CC_MEMSET, st); FORWARD(d, v, n, st);
}
hipError_t hipMemsetD8(hipDeviceptr_t d, unsigned char v, size_t n) { RESOLVE(hipMemsetD8); note_on(CC_MEMSET, NULL); FORWARD(d, v, n); }
hipError_t hipMemsetD8Async(hipDeviceptr_t d, unsigned char v, size_t n, hipStream_t st) {
  RESOLVE(hipMemsetD8Async); note_on(CC_MEMSET, st); FORWARD(d, v, n, st);
}
hipError_t hipMemsetD16(hipDeviceptr_t d, unsigned short v, size_t n) { RESOLVE(hipMemsetD16); note_on(CC_MEMSET, NULL); FORWARD(d, v, n); }
hipError_t hipMemsetD16Async(hipDeviceptr_t d, unsigned short v, size_t n, hipStream_t st) {
  RESOLVE(hipMemsetD16Async); note_on(CC_MEMSET, st); FORWARD(d, v, n, st);
}
hipError_t hipMemsetD32(hipDeviceptr_t d, int v, size_t n) { RESOLVE(hipMemsetD32); note_on(CC_MEMSET, NULL); FORWARD(d, v, n); }
hipError_t hipMemsetD32Async(hipDeviceptr_t d, int v, size_t n, hipStream_t st) {
  RESOLVE(hipMemsetD32Async); note_on(CC_MEMSET, st); FORWARD(d, v, n, st);
}

/* ---- synchronisation ---- */
hipError_t hipDeviceSynchronize(void) { RESOLVE(hipDeviceSynchronize); note(CC_DEVICE_SYNC); FORWARD(); }
hipError_t hipStreamSynchronize(hipStream_t st) {
  RESOLVE(hipStreamSynchronize);
  note(st == NULL || st == hipStreamLegacy ? CC_DEVICE_SYNC : CC_STREAM_SYNC);
  FORWARD(st);
}

/* ---- launches ---- */
hipError_t hipLaunchKernel(const void* f, dim3 g, dim3 b, void** a, size_t sm, hipStream_t st) {
  RESOLVE(hipLaunchKernel); note_on(CC_LAUNCH, st); FORWARD(f, g, b, a, sm, st);
}
hipError_t hipExtLaunchKernel(const void* f, dim3 g, dim3 b, void** a, size_t sm, hipStream_t st, hipEvent_t e0,
                              hipEvent_t e1, int flags) {
  RESOLVE(hipExtLaunchKernel); note_on(CC_LAUNCH, st); FORWARD(f, g, b, a, sm, st, e0, e1, flags);
}
hipError_t hipLaunchCooperativeKernel(const void* f, dim3 g, dim3 b, void** a, unsigned sm, hipStream_t st) {
  RESOLVE(hipLaunchCooperativeKernel); note_on(CC_LAUNCH, st); FORWARD(f, g, b, a, sm, st);
}
hipError_t hipLaunchKernelExC(const hipLaunchConfig_t* c, const void* f, void** a) {
  RESOLVE(hipLaunchKernelExC); note_on(CC_LAUNCH, c ? c->stream : NULL); FORWARD(c, f, a);
}
hipError_t hipModuleLaunchKernel(hipFunction_t f, unsigned gx, unsigned gy, unsigned gz, unsigned bx, unsigned by,
                                 unsigned bz, unsigned sm, hipStream_t st, void** a, void** extra) {
  RESOLVE(hipModuleLaunchKernel); note_on(CC_LAUNCH, st); FORWARD(f, gx, gy, gz, bx, by, bz, sm, st, a, extra);
}
hipError_t hipGraphLaunch(hipGraphExec_t g, hipStream_t st) {
  RESOLVE(hipGraphLaunch); note_on(CC_LAUNCH, st); FORWARD(g, st);
}
