/* A plain C caller of libtaskops.so: include/taskops.h and the HIP runtime API, no C++ and
 * no Python.  It runs reward_to_go on a small batch with done flags, on a created stream,
 * checks every element against the recurrence of tasks/reward_to_go/reference.py:34-42
 * evaluated in double on the host (within the task's atol = rtol = 1e-5), and checks that a
 * negative size is refused.  Prints "ok" and exits 0 on success.  Built and run by
 * tests/test_c_abi.py. */
#include <math.h>
#include <stdbool.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "taskops.h"

#define CHECK(call)                                                              \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess) {                                                      \
      fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));          \
      return 1;                                                                  \
    }                                                                            \
  } while (0)

int main(void) {
  enum { B = 37, T = 1031 };
  const float gamma = 0.97f;
  const size_t n = (size_t)B * T;
  float* reward = malloc(n * sizeof(float));
  bool* done = malloc(n * sizeof(bool));
  float* out = malloc(n * sizeof(float));
  if (!reward || !done || !out) return 1;
  uint32_t s = 12345u;
  for (size_t i = 0; i < n; ++i) {
    s = s * 1664525u + 1013904223u;
    reward[i] = (float)(s >> 8) / 16777216.0f;
    done[i] = ((s >> 4) & 63u) == 0u;
  }

  float *d_reward = NULL, *d_out = NULL;
  bool* d_done = NULL;
  hipStream_t stream = NULL;
  CHECK(hipMalloc((void**)&d_reward, n * sizeof(float)));
  CHECK(hipMalloc((void**)&d_done, n * sizeof(bool)));
  CHECK(hipMalloc((void**)&d_out, n * sizeof(float)));
  CHECK(hipStreamCreate(&stream));
  CHECK(hipMemcpy(d_reward, reward, n * sizeof(float), hipMemcpyHostToDevice));
  CHECK(hipMemcpy(d_done, done, n * sizeof(bool), hipMemcpyHostToDevice));
  CHECK(taskops_reward_to_go(d_reward, d_done, gamma, B, T, d_out, stream));
  CHECK(hipStreamSynchronize(stream));
  CHECK(hipMemcpy(out, d_out, n * sizeof(float), hipMemcpyDeviceToHost));

  size_t bad = 0;
  for (int b = 0; b < B; ++b) {
    double next = 0.0;
    for (int t = T - 1; t >= 0; --t) {
      const size_t i = (size_t)b * T + t;
      next = (double)reward[i] + (double)gamma * (done[i] ? 0.0 : next);
      if (fabs((double)out[i] - next) > 1e-5 + 1e-5 * fabs(next)) ++bad;
    }
  }
  if (taskops_pow_abs_sqrt_mean(NULL, NULL, -1, 1, 1, NULL, stream) != hipErrorInvalidValue) {
    fprintf(stderr, "a negative size was not refused\n");
    return 1;
  }
  CHECK(hipStreamDestroy(stream));
  CHECK(hipFree(d_reward));
  CHECK(hipFree(d_done));
  CHECK(hipFree(d_out));
  free(reward);
  free(done);
  free(out);
  if (bad) {
    fprintf(stderr, "%zu of %zu outputs outside the tolerance\n", bad, n);
    return 1;
  }
  printf("ok\n");
  return 0;
}
