// PyTorch operators over the C ABI of include/taskops.h: torch.ops.taskops.<op>.
//
// Each operator checks its tensors (device, dtype, contiguity, shapes), allocates its
// outputs with the caching allocator, calls the taskops_* entry point on the current HIP
// stream of the input's device, and turns a non-zero hipError_t into an error
// (TORCH_CHECK).  Meta kernels give the output shapes for tracing.  Host code only: the
// kernels are in libtaskops.so, which this library links.
//
// Operators, with the reference computation each one replaces:
//   pow_abs_sqrt_mean(inp, target) -> 0-d          tasks/pow_abs_sqrt_mean/reference.py:22-28
//   leaky(input_current, mem0, beta, threshold) -> (spikes, final_mem)   tasks/leaky/reference.py:26-37
//   reward_to_go(reward, done, gamma) -> output    tasks/reward_to_go/reference.py:22-31
//   ppo_clip(cur, old, adv, clip_epsilon) -> [6]   tasks/ppo_clip/reference.py:27-39
//   ppo_clip_entropy(cur, old, adv, entropy, clip_epsilon, entropy_coef) -> [8]
//   efficient_kan(x, grid, base_weight, spline_weight, spline_scaler, grid_size, spline_order) -> out
//                                                  tasks/efficient_kan/reference.py:42-51
//   fp8_linear(x_fp8, scale_x, w_fp8, scale_w, bias) -> bf16 output   tasks/fp8_linear/reference.py:34-41
//   quantize_e4m3(x) -> (q e4m3, scale fp32[1])    tasks/fp8_linear/reference.py:15-18
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include "taskops.h"

namespace {

using at::Tensor;

// ROCm builds of torch present HIP devices as device type "cuda"; the masquerading guard
// and stream accept them.
using DeviceGuard = c10::hip::HIPGuardMasqueradingAsCUDA;

hipStream_t stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

void check(hipError_t e, const char* what) {
  TORCH_CHECK(e == hipSuccess, what, " failed: hipError_t ", static_cast<int>(e), " (", hipGetErrorString(e), ")");
}

void expect(const Tensor& t, const char* name, at::ScalarType dtype, const Tensor& like) {
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
  TORCH_CHECK(t.device() == like.device(), name, " must be on ", like.device());
  TORCH_CHECK(t.scalar_type() == dtype, name, " must be ", dtype, ", got ", t.scalar_type());
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

template <class T>
T* ptr(const Tensor& t) {
  return reinterpret_cast<T*>(t.data_ptr());
}

int32_t as_i32(int64_t v, const char* name) {
  TORCH_CHECK(v >= 0 && v <= INT32_MAX, name, " = ", v, " does not fit the entry point's int32_t");
  return static_cast<int32_t>(v);
}

// ---- pow_abs_sqrt_mean: inp, target of shape [B, 4, H, W] ----
void pow_shape(const Tensor& inp, const Tensor& target) {
  TORCH_CHECK(inp.dim() == 4 && inp.size(1) == 4, "inp must be [B, 4, H, W]");
  TORCH_CHECK(target.sizes() == inp.sizes(), "target must match inp's shape");
}
Tensor pow_abs_sqrt_mean_gpu(const Tensor& inp, const Tensor& target) {
  pow_shape(inp, target);
  expect(inp, "inp", at::kFloat, inp);
  expect(target, "target", at::kFloat, inp);
  DeviceGuard guard(inp.device());
  Tensor out = at::empty({}, inp.options());
  check(taskops_pow_abs_sqrt_mean(ptr<const float>(inp), ptr<const float>(target), inp.size(0), inp.size(2),
                                  inp.size(3), ptr<float>(out), stream_of(inp)),
        "taskops_pow_abs_sqrt_mean");
  return out;
}
Tensor pow_abs_sqrt_mean_meta(const Tensor& inp, const Tensor& target) {
  pow_shape(inp, target);
  return at::empty({}, inp.options());
}

// ---- leaky: input_current [T, B, H], mem0 [B, H], beta [H], threshold [H] ----
void leaky_shape(const Tensor& x, const Tensor& mem0, const Tensor& beta, const Tensor& th) {
  TORCH_CHECK(x.dim() == 3, "input_current must be [T, B, H]");
  TORCH_CHECK(mem0.dim() == 2 && mem0.size(0) == x.size(1) && mem0.size(1) == x.size(2), "mem0 must be [B, H]");
  TORCH_CHECK(beta.numel() == x.size(2) && th.numel() == x.size(2), "beta and threshold must have H elements");
}
std::tuple<Tensor, Tensor> leaky_gpu(const Tensor& x, const Tensor& mem0, const Tensor& beta, const Tensor& th) {
  leaky_shape(x, mem0, beta, th);
  expect(x, "input_current", at::kFloat, x);
  expect(mem0, "mem0", at::kFloat, x);
  expect(beta, "beta", at::kFloat, x);
  expect(th, "threshold", at::kFloat, x);
  DeviceGuard guard(x.device());
  Tensor spikes = at::empty_like(x), fin = at::empty_like(mem0);
  check(taskops_leaky(ptr<const float>(x), ptr<const float>(mem0), ptr<const float>(beta), ptr<const float>(th),
                      as_i32(x.size(0), "T"), as_i32(x.size(1), "B"), as_i32(x.size(2), "H"), ptr<float>(spikes),
                      ptr<float>(fin), stream_of(x)),
        "taskops_leaky");
  return {spikes, fin};
}
std::tuple<Tensor, Tensor> leaky_meta(const Tensor& x, const Tensor& mem0, const Tensor& beta, const Tensor& th) {
  leaky_shape(x, mem0, beta, th);
  return {at::empty_like(x), at::empty_like(mem0)};
}

// ---- reward_to_go: reward [B, T] fp32, done [B, T] bool ----
void rtg_shape(const Tensor& reward, const Tensor& done) {
  TORCH_CHECK(reward.dim() == 2, "reward must be [B, T]");
  TORCH_CHECK(done.sizes() == reward.sizes(), "done must match reward's shape");
}
Tensor reward_to_go_gpu(const Tensor& reward, const Tensor& done, double gamma) {
  rtg_shape(reward, done);
  expect(reward, "reward", at::kFloat, reward);
  expect(done, "done", at::kBool, reward);
  DeviceGuard guard(reward.device());
  Tensor out = at::empty_like(reward);
  check(taskops_reward_to_go(ptr<const float>(reward), ptr<const bool>(done), static_cast<float>(gamma),
                             as_i32(reward.size(0), "B"), as_i32(reward.size(1), "T"), ptr<float>(out),
                             stream_of(reward)),
        "taskops_reward_to_go");
  return out;
}
Tensor reward_to_go_meta(const Tensor& reward, const Tensor& done, double) {
  rtg_shape(reward, done);
  return at::empty_like(reward);
}

// ---- ppo_clip: three (or four) tensors [B, T, H] ----
void ppo_shape(const Tensor& cur, const Tensor& old, const Tensor& adv) {
  TORCH_CHECK(cur.dim() == 3, "current_log_prob must be [B, T, H]");
  TORCH_CHECK(old.sizes() == cur.sizes() && adv.sizes() == cur.sizes(), "old_log_prob and advantage must match");
}
Tensor ppo_clip_gpu(const Tensor& cur, const Tensor& old, const Tensor& adv, double eps) {
  ppo_shape(cur, old, adv);
  expect(cur, "current_log_prob", at::kFloat, cur);
  expect(old, "old_log_prob", at::kFloat, cur);
  expect(adv, "advantage", at::kFloat, cur);
  DeviceGuard guard(cur.device());
  Tensor out = at::empty({6}, cur.options());
  check(taskops_ppo_clip(as_i32(cur.size(0), "B"), as_i32(cur.size(1), "T"), as_i32(cur.size(2), "H"),
                         ptr<const float>(cur), ptr<const float>(old), ptr<const float>(adv), static_cast<float>(eps),
                         ptr<float>(out), stream_of(cur)),
        "taskops_ppo_clip");
  return out;
}
Tensor ppo_clip_meta(const Tensor& cur, const Tensor& old, const Tensor& adv, double) {
  ppo_shape(cur, old, adv);
  return at::empty({6}, cur.options());
}
Tensor ppo_clip_entropy_gpu(const Tensor& cur, const Tensor& old, const Tensor& adv, const Tensor& ent, double eps,
                            double coef) {
  ppo_shape(cur, old, adv);
  TORCH_CHECK(ent.sizes() == cur.sizes(), "entropy must match current_log_prob");
  expect(cur, "current_log_prob", at::kFloat, cur);
  expect(old, "old_log_prob", at::kFloat, cur);
  expect(adv, "advantage", at::kFloat, cur);
  expect(ent, "entropy", at::kFloat, cur);
  DeviceGuard guard(cur.device());
  Tensor out = at::empty({8}, cur.options());
  check(taskops_ppo_clip_entropy(as_i32(cur.size(0), "B"), as_i32(cur.size(1), "T"), as_i32(cur.size(2), "H"),
                                 ptr<const float>(cur), ptr<const float>(old), ptr<const float>(adv),
                                 ptr<const float>(ent), static_cast<float>(eps), static_cast<float>(coef),
                                 ptr<float>(out), stream_of(cur)),
        "taskops_ppo_clip_entropy");
  return out;
}
Tensor ppo_clip_entropy_meta(const Tensor& cur, const Tensor& old, const Tensor& adv, const Tensor& ent, double,
                             double) {
  ppo_shape(cur, old, adv);
  TORCH_CHECK(ent.sizes() == cur.sizes(), "entropy must match current_log_prob");
  return at::empty({8}, cur.options());
}

// ---- efficient_kan: x [B, I], grid [I, G + 2K + 1], Wb [O, I], Ws [O, I, G + K], scaler [O, I] ----
void kan_shape(const Tensor& x, const Tensor& grid, const Tensor& wb, const Tensor& ws, const Tensor& sc,
               int64_t G, int64_t K) {
  TORCH_CHECK(G >= 1 && K >= 0, "grid_size must be >= 1 and spline_order >= 0");
  TORCH_CHECK(x.dim() == 2, "x must be [B, I]");
  const int64_t I = x.size(1);
  TORCH_CHECK(grid.dim() == 2 && grid.size(0) == I && grid.size(1) == G + 2 * K + 1, "grid must be [I, G + 2K + 1]");
  TORCH_CHECK(wb.dim() == 2 && wb.size(1) == I, "base_weight must be [O, I]");
  TORCH_CHECK(ws.dim() == 3 && ws.size(0) == wb.size(0) && ws.size(1) == I && ws.size(2) == G + K,
              "spline_weight must be [O, I, G + K]");
  TORCH_CHECK(sc.sizes() == wb.sizes(), "spline_scaler must be [O, I]");
}
Tensor efficient_kan_gpu(const Tensor& x, const Tensor& grid, const Tensor& wb, const Tensor& ws, const Tensor& sc,
                         int64_t G, int64_t K) {
  kan_shape(x, grid, wb, ws, sc, G, K);
  for (auto p : {std::make_pair(&x, "x"), std::make_pair(&grid, "grid"), std::make_pair(&wb, "base_weight"),
                 std::make_pair(&ws, "spline_weight"), std::make_pair(&sc, "spline_scaler")})
    expect(*p.first, p.second, at::kFloat, x);
  DeviceGuard guard(x.device());
  Tensor out = at::empty({x.size(0), wb.size(0)}, x.options());
  check(taskops_efficient_kan(ptr<const float>(x), ptr<const float>(grid), ptr<const float>(wb), ptr<const float>(ws),
                              ptr<const float>(sc), as_i32(G, "grid_size"), as_i32(K, "spline_order"),
                              as_i32(x.size(0), "B"), as_i32(x.size(1), "I"), as_i32(wb.size(0), "O"), ptr<float>(out),
                              stream_of(x)),
        "taskops_efficient_kan");
  return out;
}
Tensor efficient_kan_meta(const Tensor& x, const Tensor& grid, const Tensor& wb, const Tensor& ws, const Tensor& sc,
                          int64_t G, int64_t K) {
  kan_shape(x, grid, wb, ws, sc, G, K);
  return at::empty({x.size(0), wb.size(0)}, x.options());
}

// ---- fp8_linear: x [M, K] e4m3, w [N, K] e4m3, bias [N] bf16 -> [M, N] bf16 ----
void fp8_shape(const Tensor& x, const Tensor& w, const Tensor& bias) {
  TORCH_CHECK(x.dim() == 2 && w.dim() == 2 && x.size(1) == w.size(1), "x must be [M, K] and w [N, K]");
  TORCH_CHECK(bias.dim() == 1 && bias.size(0) == w.size(0), "bias must be [N]");
}
Tensor fp8_linear_gpu(const Tensor& x, double scale_x, const Tensor& w, double scale_w, const Tensor& bias) {
  fp8_shape(x, w, bias);
  expect(x, "x_fp8", at::kFloat8_e4m3fn, x);
  expect(w, "w_fp8", at::kFloat8_e4m3fn, x);
  expect(bias, "bias", at::kBFloat16, x);
  DeviceGuard guard(x.device());
  Tensor out = at::empty({x.size(0), w.size(0)}, x.options().dtype(at::kBFloat16));
  check(taskops_fp8_linear(as_i32(x.size(0), "M"), as_i32(x.size(1), "K"), as_i32(w.size(0), "N"), ptr<const uint8_t>(x),
                           static_cast<float>(scale_x), ptr<const uint8_t>(w), static_cast<float>(scale_w),
                           ptr<const uint16_t>(bias), ptr<uint16_t>(out), stream_of(x)),
        "taskops_fp8_linear");
  return out;
}
Tensor fp8_linear_meta(const Tensor& x, double, const Tensor& w, double, const Tensor& bias) {
  fp8_shape(x, w, bias);
  return at::empty({x.size(0), w.size(0)}, x.options().dtype(at::kBFloat16));
}

// ---- quantize_e4m3: any contiguous fp32 tensor -> same-shape e4m3 codes + fp32 scale [1] ----
// An empty x is an error, as the reference's x.abs().max() is.
std::tuple<Tensor, Tensor> quantize_e4m3_gpu(const Tensor& x) {
  expect(x, "x", at::kFloat, x);
  TORCH_CHECK(x.numel() > 0, "quantize_e4m3: an empty tensor has no max |x|");
  DeviceGuard guard(x.device());
  Tensor q = at::empty(x.sizes(), x.options().dtype(at::kFloat8_e4m3fn));
  Tensor scale = at::empty({1}, x.options());
  check(taskops_quantize_e4m3(ptr<const float>(x), x.numel(), ptr<uint8_t>(q), ptr<float>(scale), stream_of(x)),
        "taskops_quantize_e4m3");
  return {q, scale};
}
std::tuple<Tensor, Tensor> quantize_e4m3_meta(const Tensor& x) {
  TORCH_CHECK(x.numel() > 0, "quantize_e4m3: an empty tensor has no max |x|");
  return {at::empty(x.sizes(), x.options().dtype(at::kFloat8_e4m3fn)), at::empty({1}, x.options())};
}

}  // namespace

TORCH_LIBRARY(taskops, m) {
  m.def("pow_abs_sqrt_mean(Tensor inp, Tensor target) -> Tensor");
  m.def("leaky(Tensor input_current, Tensor mem0, Tensor beta, Tensor threshold) -> (Tensor, Tensor)");
  m.def("reward_to_go(Tensor reward, Tensor done, float gamma) -> Tensor");
  m.def("ppo_clip(Tensor current_log_prob, Tensor old_log_prob, Tensor advantage, float clip_epsilon) -> Tensor");
  m.def(
      "ppo_clip_entropy(Tensor current_log_prob, Tensor old_log_prob, Tensor advantage, Tensor entropy, "
      "float clip_epsilon, float entropy_coef) -> Tensor");
  m.def(
      "efficient_kan(Tensor x, Tensor grid, Tensor base_weight, Tensor spline_weight, Tensor spline_scaler, "
      "int grid_size, int spline_order) -> Tensor");
  m.def("fp8_linear(Tensor x_fp8, float scale_x, Tensor w_fp8, float scale_w, Tensor bias) -> Tensor");
  m.def("quantize_e4m3(Tensor x) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(taskops, CUDA, m) {
  m.impl("pow_abs_sqrt_mean", &pow_abs_sqrt_mean_gpu);
  m.impl("leaky", &leaky_gpu);
  m.impl("reward_to_go", &reward_to_go_gpu);
  m.impl("ppo_clip", &ppo_clip_gpu);
  m.impl("ppo_clip_entropy", &ppo_clip_entropy_gpu);
  m.impl("efficient_kan", &efficient_kan_gpu);
  m.impl("fp8_linear", &fp8_linear_gpu);
  m.impl("quantize_e4m3", &quantize_e4m3_gpu);
}

TORCH_LIBRARY_IMPL(taskops, Meta, m) {
  m.impl("pow_abs_sqrt_mean", &pow_abs_sqrt_mean_meta);
  m.impl("leaky", &leaky_meta);
  m.impl("reward_to_go", &reward_to_go_meta);
  m.impl("ppo_clip", &ppo_clip_meta);
  m.impl("ppo_clip_entropy", &ppo_clip_entropy_meta);
  m.impl("efficient_kan", &efficient_kan_meta);
  m.impl("fp8_linear", &fp8_linear_meta);
  m.impl("quantize_e4m3", &quantize_e4m3_meta);
}
