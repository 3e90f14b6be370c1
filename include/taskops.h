/*
 * taskops.h — C ABI of the MI355X (gfx950) task-op library `libtaskops.so`.
 *
 * Each entry point replaces one task op of Mohamed-Alaboudi/cuda-optimization-benchmark,
 * whose public interface is a C++ `void reference(...)` per task (the signature in
 * tasks/<id>/tests/task.json:3, implemented by reference/<id>/solution.cu).  The
 * arguments keep that signature's order, meaning and scalar types; two things are added:
 *
 *   - the HIP stream the work is enqueued on (NULL = the default stream, as the
 *     reference's prompts require: "Launch your work on the default stream");
 *   - a return value: hipSuccess (0) or the hipError_t of the failed launch or argument
 *     check.  The reference's `void` entry has no error channel (errors surface at the
 *     caller's next synchronize); the C++ drop-in overloads in dropin.hpp keep `void`.
 *
 * All pointers are device pointers to contiguous row-major data, owned by the caller.
 * The library keeps one cached workspace per device and op family (allocated on the first
 * call that needs it, grown when a call needs more, never freed before exit; efficient_kan's
 * holds the packed weights, about 38.5 MB at B = 8192, I = O = 1024) and never caches
 * results or derived weight contents between calls.  Calls are asynchronous: no host synchronisation and no
 * device-to-host copy happens inside a call.  Calls that share a device and overlap in
 * time on different streams race on that workspace (as the reference's statics do);
 * calls on one stream are safe.
 *
 * Raw-bit types are used at the boundary for the two non-C element types:
 *   e4m3 (OCP FP8, 1 byte)  -> uint8_t   (the reference uses __nv_fp8_e4m3)
 *   bfloat16 (2 bytes)      -> uint16_t  (the reference uses __nv_bfloat16)
 */
#ifndef TASKOPS_H_
#define TASKOPS_H_

#include <hip/hip_runtime_api.h>
#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library version; bumps when an entry point's behaviour changes. */
int taskops_version(void);

/* output[0] = mean over n = batch_size*4*height*width elements of
 * sqrt((inp - target)^2 + 1e-6), fp32 result of an fp64 reduction.  n == 0 writes NaN
 * (the mean of nothing, as reference_exact gives); a negative dimension, or n above 2^40,
 * returns hipErrorInvalidValue and writes nothing.
 * Replaces: reference/pow_abs_sqrt_mean/solution.cu:99-118
 *           (tasks/pow_abs_sqrt_mean/tests/task.json:3; op: reference.py:22-28). */
hipError_t taskops_pow_abs_sqrt_mean(const float* inp, const float* target,
                                     int64_t batch_size, int64_t height, int64_t width,
                                     float* output, hipStream_t stream);

/* Leaky integrate-and-fire layer, reset by subtraction, T steps over B*H neurons.
 * beta is clamped to [0,1]; per step: reset = (mem >= th); mem = beta*mem + x[t] - reset*th
 * (each operation rounded in fp32, no contraction); spikes[t] = (mem >= th).
 * Bit-identical to the fp32 step-by-step reference.  Negative sizes, or B*H above
 * 2^32 - 256 neurons (one launch's work-items), return hipErrorInvalidValue.
 * Replaces: reference/leaky/solution.cu:106-138 (tasks/leaky/tests/task.json:3;
 *           op: tasks/leaky/reference.py:26-37). */
hipError_t taskops_leaky(const float* input_current, const float* mem0, const float* beta,
                         const float* threshold, int32_t T, int32_t B, int32_t H,
                         float* spikes, float* final_mem, hipStream_t stream);

/* output[b,t] = reward[b,t] + gamma * (done[b,t] ? 0 : output[b,t+1]), output[b,T] = 0.
 * Affine scan carried in fp64, one rounding to fp32 per element.  B <= 0 or T <= 0 does
 * nothing.  Any T up to INT32_MAX; rows of 2^30 steps or more take the element-wise path.
 * Replaces: reference/reward_to_go/solution.cu:237-264
 *           (tasks/reward_to_go/tests/task.json:3; op: reference.py:34-42). */
hipError_t taskops_reward_to_go(const float* reward, const bool* done, float gamma,
                                int32_t B, int32_t T, float* output, hipStream_t stream);

/* PPO clipped objective and metrics over N = B*T*H samples, one pass, one launch.
 * output[0..5] = [loss_objective, clip_fraction, approx_kl, ess, max_ratio, mean_ratio].
 * B, T or H <= 0, or B*T*H above 2^40, returns hipErrorInvalidValue and writes nothing.
 * Replaces: reference/ppo_clip/solution.cu:165-182 (tasks/ppo_clip/tests/task.json:3;
 *           op: tasks/ppo_clip/reference.py:27-39). */
hipError_t taskops_ppo_clip(int32_t B, int32_t T, int32_t H, const float* current_log_prob,
                            const float* old_log_prob, const float* advantage,
                            float clip_epsilon, float* output, hipStream_t stream);

/* The same single pass, also reading a per-sample entropy:
 * output[0..7] = [loss_objective, clip_fraction, approx_kl, ess, max_ratio, mean_ratio,
 *                 mean_entropy, loss_entropy = -entropy_coef * mean_entropy].
 * Has no counterpart in the reference; it is the ClipPPOLoss entropy bonus term that the
 * benchmark's BASELINE configuration adds (TorchRL ClipPPOLoss, entropy_coef). */
hipError_t taskops_ppo_clip_entropy(int32_t B, int32_t T, int32_t H,
                                    const float* current_log_prob, const float* old_log_prob,
                                    const float* advantage, const float* entropy,
                                    float clip_epsilon, float entropy_coef, float* output,
                                    hipStream_t stream);

/* taskops_ppo_clip_entropy without any allocation: the same kernel, launch shape and result
 * bits, with the reduction's scratch (per-workgroup records and arrival counters) in a
 * fixed 263,232-byte device array of the library instead of a workspace allocated on the
 * first call.  No counterpart in the reference: it is for callers that cannot call
 * hipMalloc (code under HIP graph capture, serving loops, harnesses that forbid it).
 * Every call on one GPU shares that GPU's array, so calls that overlap in time on one GPU
 * (different streams, or host threads) race; calls on one stream are safe.  The first call
 * on a device clears the array with a kernel on `stream`.  Any B*T*H up to 2^40 samples
 * fits; larger products and B, T or H <= 0 return hipErrorInvalidValue and write nothing. */
hipError_t taskops_ppo_clip_entropy_noalloc(int32_t B, int32_t T, int32_t H,
                                            const float* current_log_prob,
                                            const float* old_log_prob, const float* advantage,
                                            const float* entropy, float clip_epsilon,
                                            float entropy_coef, float* output,
                                            hipStream_t stream);

/* KANLinear forward: out[B,O] = silu(x) @ base_weight^T
 *                              + bsplines(x; grid) @ (spline_weight * spline_scaler[...,None])^T
 * grid is [I, grid_size + 2*spline_order + 1] (per-feature knots, strictly increasing),
 * spline_weight is [O, I, grid_size + spline_order].  fp32 in and out.
 * Spline order 3 with at most 16 knots per feature takes the fp16x3 MFMA path, whose limits
 * are: |x| < 65504 (silu(x) is carried in fp16 halves); within one output column the
 * nonzero entries of base_weight and spline_weight*spline_scaler span at most about 2^24
 * in magnitude (smaller ones lose bits to the fp16 low halves); knot rows uniform to
 * 5e-7 h use the cardinal cubic pieces (about 1e-6 of a basis value from the exact bases),
 * all other rows exact per-interval cubics.  It also needs x, out, its packed weights and
 * two output columns' I x 16 spline slots each under 2 GiB (spline_weight as a whole may be
 * larger).  Other orders, knot counts and sizes take an fp32 row-wise path without these
 * limits.
 * Replaces: reference/efficient_kan/solution.cu:177-288
 *           (tasks/efficient_kan/tests/task.json:3; op: reference.py:33-51). */
hipError_t taskops_efficient_kan(const float* x, const float* grid, const float* base_weight,
                                 const float* spline_weight, const float* spline_scaler,
                                 int32_t grid_size, int32_t spline_order, int32_t B, int32_t I,
                                 int32_t O, float* out, hipStream_t stream);

/* FP8 (OCP e4m3) linear: output[M,N] = bf16( (x/scale_x) @ (w/scale_w)^T + bias ),
 * x [M,K] and w [N,K] row-major e4m3 bytes, bias [N] bf16, fp32 accumulation, one
 * round-to-nearest-even to bf16.  A workgroup addresses its rows with 32-bit offsets, so
 * shapes past them return hipErrorInvalidValue and write nothing: for M > 64, K above
 * 8,388,607 or N above 4,194,303; for M <= 64, M*K or 16*K above 2^31 - 1, or N above
 * 134,217,727 (one launch's work-items).  Negative
 * sizes return hipErrorInvalidValue; M == 0 or N == 0 does nothing.
 * Replaces: reference/fp8_linear/solution.cu:276-321 (tasks/fp8_linear/tests/task.json:3;
 *           op: tasks/fp8_linear/reference.py:34-41). */
hipError_t taskops_fp8_linear(int32_t M, int32_t K, int32_t N, const uint8_t* x_fp8,
                              float scale_x, const uint8_t* w_fp8, float scale_w,
                              const uint16_t* bias, uint16_t* output, hipStream_t stream);

/* Per-tensor max-abs OCP e4m3 quantisation of x[n] (fp32), the step that produces
 * fp8_linear's operands: *scale = fp32(448 / max(max|x|, 1e-9)) with the quotient in fp64,
 * q[i] = e4m3(clamp(x[i] * *scale, -448, 448)), round to nearest even; a NaN in x makes
 * *scale and every q[i] NaN (0x7F or 0xFF: the sign of a computed NaN is unspecified).
 * q and scale are device pointers.  n == 0 writes nothing;
 * n < 0 returns hipErrorInvalidValue.  Aligned x (16 B) and q (4 B) up to the resident
 * capacity (1280 chunks of 16384 elements on an MI355X) take one launch with a bounded grid
 * barrier; other calls take two launches.  Both give the same bits.
 * Replaces: tasks/fp8_linear/reference.py:15-18 (`_quantize`, which the reference runs on
 *           the CPU before the op). */
hipError_t taskops_quantize_e4m3(const float* x, int64_t n, uint8_t* q, float* scale,
                                 hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TASKOPS_H_ */
