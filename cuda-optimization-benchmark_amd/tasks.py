"""The six task specifications: signature, outputs, tolerance and input cases.

Facts restated from the benchmark's task files (tasks/<id>/tests/task.json, the hidden
cases; tasks/<id>/environment/public_cases.json, the two public cases) and the BASELINE
configurations this build is measured on.  `signature` is the reference's C++ entry
verbatim; `hip_signature` is the same with the two CUDA element types replaced by HIP's
ABI-identical ones.
"""
from __future__ import annotations

import copy

SET_B = 7919  # call 2 uses seed + SET_B (graders/grade.py:45)

_SIG = {
    "pow_abs_sqrt_mean": "void reference(const float* inp, const float* target, int64_t batch_size, "
                         "int64_t height, int64_t width, float* output);",
    "leaky": "void reference(const float* input_current, const float* mem0, const float* beta, "
             "const float* threshold, int32_t T, int32_t B, int32_t H, float* spikes, float* final_mem);",
    "reward_to_go": "void reference(const float* reward, const bool* done, float gamma, int32_t B, "
                    "int32_t T, float* output);",
    "ppo_clip": "void reference(const int32_t B, const int32_t T, const int32_t H, const float* "
                "current_log_prob, const float* old_log_prob, const float* advantage, const float "
                "clip_epsilon, float* output);",
    "efficient_kan": "void reference(const float* x, const float* grid, const float* base_weight, "
                     "const float* spline_weight, const float* spline_scaler, int32_t grid_size, "
                     "int32_t spline_order, int32_t B, int32_t I, int32_t O, float* out);",
    "fp8_linear": "void reference(const int32_t M, const int32_t K, const int32_t N, const "
                  "__nv_fp8_e4m3* x_fp8, float scale_x, const __nv_fp8_e4m3* w_fp8, float scale_w, "
                  "const __nv_bfloat16* bias, __nv_bfloat16* output);",
}

_OUT = {
    "pow_abs_sqrt_mean": {"output": {"dtype": "float32", "shape": []}},
    "leaky": {"spikes": {"dtype": "float32", "shape": ["T", "B", "H"]},
              "final_mem": {"dtype": "float32", "shape": ["B", "H"]}},
    "reward_to_go": {"output": {"dtype": "float32", "shape": ["B", "T"]}},
    "ppo_clip": {"output": {"dtype": "float32", "shape": [6]}},
    "efficient_kan": {"out": {"dtype": "float32", "shape": ["B", "O"]}},
    "fp8_linear": {"output": {"dtype": "bfloat16", "shape": ["M", "N"]}},
}

_TOL = {
    "pow_abs_sqrt_mean": {"atol": 1e-3, "rtol": 1e-3},
    "leaky": {"atol": 1e-6, "rtol": 1e-5},
    "reward_to_go": {"atol": 1e-5, "rtol": 1e-5},
    "ppo_clip": {"atol": 1e-5, "rtol": 1e-4},
    "efficient_kan": {"atol": 1e-5, "rtol": 1e-5},
    "fp8_linear": {"atol": 1e-2, "rtol": 1e-2},
}


def _c(name, seed, small=False, timed=False, **kw):
    return dict(name=name, seed=seed, small=small, timed=timed, **kw)


# Hidden cases (tests/task.json "cases").
_HIDDEN = {
    "pow_abs_sqrt_mean": [
        _c("b4_h4_w4", 101, batch_size=4, height=4, width=4),
        _c("b16_h4_w8", 102, batch_size=16, height=4, width=8),
        _c("b1_h1_w1", 103, batch_size=1, height=1, width=1),
        _c("b3_h129_w257", 104, small=True, batch_size=3, height=129, width=257),
        _c("b8_h64_w64_scale1000", 105, batch_size=8, height=64, width=64, scale=1000.0),
        _c("b16_h512_w512", 106, timed=True, batch_size=16, height=512, width=512),
    ],
    "leaky": [
        _c("T1_B1_H1021", 201, T=1, B=1, H=1021),
        _c("T33_B65_H129_mem0", 202, small=True, T=33, B=65, H=129, mem0_std=0.1),
        _c("T160_B85_H200", 203, T=160, B=85, H=200),
        _c("T32_B64_H128_beta_out_of_range", 204, T=32, B=64, H=128, beta_range=[-0.2, 1.2]),
        _c("T256_B512_H1024", 205, timed=True, T=256, B=512, H=1024),
    ],
    "reward_to_go": [
        _c("B3_T1", 601, B=3, T=1, gamma=0.5, done_p=0.1),
        _c("B7_T999", 602, small=True, B=7, T=999, gamma=0.9, done_p=0.1),
        _c("B256_T1024", 603, B=256, T=1024, gamma=0.99, done_p=0.01),
        _c("B1_T8000", 604, B=1, T=8000, gamma=0.99, done_p=0.001),
        _c("B64_T1024", 605, timed=True, B=64, T=1024, gamma=0.99, done_p=0.1),
    ],
    "ppo_clip": [
        _c("B1_T1_H1", 501, B=1, T=1, H=1),
        _c("B7_T13_H3", 502, B=7, T=13, H=3),
        _c("B1000_T333_H2", 503, small=True, B=1000, T=333, H=2),
        _c("B512_T256_H1_wide", 504, B=512, T=256, H=1, delta_std=1.0, clip_epsilon=0.1),
        _c("B4096_T256_H1", 505, timed=True, B=4096, T=256, H=1),
    ],
    "efficient_kan": [
        _c("B1_I256_O512", 301, B=1, I=256, O=512),
        _c("B1000_I256_O512", 302, B=1000, I=256, O=512),
        _c("B64_I100_O300", 303, small=True, B=64, I=100, O=300),
        _c("B512_I256_O512_wide_x", 304, B=512, I=256, O=512, x_range=2.0),
        _c("B4096_I256_O512", 305, timed=True, B=4096, I=256, O=512),
    ],
    "fp8_linear": [
        _c("M1_K1024_N4096", 401, M=1, K=1024, N=4096),
        _c("M16_K64_N128", 402, small=True, M=16, K=64, N=128),
        _c("M333_K1000_N3000", 403, M=333, K=1000, N=3000),
        _c("M2048_K1024_N4096", 404, timed=True, M=2048, K=1024, N=4096),
    ],
}

# Public cases (environment/public_cases.json "cases").
_PUBLIC = {
    "pow_abs_sqrt_mean": [
        _c("b4_h4_w4", 11, small=True, batch_size=4, height=4, width=4),
        _c("b3_h7_w11", 12, small=True, batch_size=3, height=7, width=11),
    ],
    "leaky": [
        _c("T8_B4_H33", 21, small=True, T=8, B=4, H=33),
        _c("T16_B3_H65_mem0", 22, small=True, T=16, B=3, H=65, mem0_std=0.1),
    ],
    "reward_to_go": [
        _c("B4_T37", 61, small=True, B=4, T=37, gamma=0.9, done_p=0.1),
        _c("B2_T300", 62, small=True, B=2, T=300, gamma=0.99, done_p=0.01),
    ],
    "ppo_clip": [
        _c("B7_T13_H3", 51, small=True, B=7, T=13, H=3),
        _c("B4_T50_H1_wide", 52, small=True, B=4, T=50, H=1, delta_std=1.0, clip_epsilon=0.1),
    ],
    "efficient_kan": [
        _c("B8_I16_O24", 31, small=True, B=8, I=16, O=24),
        _c("B5_I7_O9_wide_x", 32, small=True, B=5, I=7, O=9, x_range=2.0),
    ],
    "fp8_linear": [
        _c("M16_K64_N128", 41, small=True, M=16, K=64, N=128),
        _c("M5_K32_N40", 42, small=True, M=5, K=32, N=40),
    ],
}

# BASELINE.json configurations (the measured workloads).  `kind: "baseline"` routes
# input generation to the BASELINE distributions in inputs.py.
BASELINE = {
    "pow_abs_sqrt_mean": _c("baseline_b16_h1024_w1024", 106, kind="baseline",
                            batch_size=16, height=1024, width=1024),
    "reward_to_go": _c("baseline_B4096_T4096", 605, kind="baseline", B=4096, T=4096,
                       gamma=0.99, done_p=0.01),
    "leaky": _c("baseline_T256_B64_H4096", 205, kind="baseline", T=256, B=64, H=4096),
    "ppo_clip": _c("baseline_B65536_T256_H1_entropy", 505, kind="baseline", B=65536, T=256, H=1,
                   clip_epsilon=0.2, entropy_coef=0.01),
    "efficient_kan": _c("baseline_B8192_I1024_O1024_G5", 305, kind="baseline", B=8192, I=1024,
                        O=1024, grid_size=5, spline_order=3),
    "fp8_linear": _c("baseline_M4096_K4096_N4096", 404, kind="baseline", M=4096, K=4096, N=4096),
    "fp8_linear_m16": _c("baseline_M16_K4096_N4096", 401, kind="baseline", M=16, K=4096, N=4096),
}

OPS = list(_SIG)


def hip_signature(sig: str) -> str:
    """The signature with the CUDA element types replaced by HIP's ABI-identical ones."""
    return sig.replace("__nv_fp8_e4m3", "__hip_fp8_e4m3").replace("__nv_bfloat16", "__hip_bfloat16")


def load_task(op: str) -> dict:
    """The task record of one op: its signature (and the parsed parameters), outputs,
    tolerance and cases."""
    from .grader.signature import parse
    t = {"task": op, "signature": _SIG[op], "outputs": copy.deepcopy(_OUT[op]),
         "tolerance": dict(_TOL[op]), "cases": copy.deepcopy(_HIDDEN[op]),
         "public_cases": copy.deepcopy(_PUBLIC[op])}
    t["hip_signature"] = hip_signature(t["signature"])
    t["params"] = parse(t["signature"])
    return t


def timed_case(op: str) -> dict:
    """The case the reference's harness times for `op` (one per task)."""
    return copy.deepcopy(next(c for c in _HIDDEN[op] if c["timed"]))


def all_cases(op: str) -> list[dict]:
    """Hidden then public cases (public names get a `public_` prefix)."""
    out = copy.deepcopy(_HIDDEN[op])
    for c in copy.deepcopy(_PUBLIC[op]):
        c["name"] = "public_" + c["name"]
        out.append(c)
    return out
