"""Seeded input generators for the six ops, on the CPU.

`make_inputs(op, case, seed)` restates each task's `make_inputs(case, seed, device)` with a
CPU `torch.Generator` and the same draw order (tasks/<id>/reference.py, cited per
function), so the same seed gives the same tensors bit for bit; tests/golden pins that
with SHA-256 digests of the reference's own tensors.  Cases with `kind: "baseline"` draw
the BASELINE.json distributions instead.  Inputs are made on the CPU (device RNG streams
differ between GPU models) and copied to the device by the caller.

The returned dict is keyed by the C argument names of the op's signature (tensors and
Python scalars); fp8 tensors are returned as `torch.float8_e4m3fn`.
"""
from __future__ import annotations

import math

import numpy as np
import torch

E4M3_MAX = 448.0


def _gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(int(seed))


def _f(g):
    return dict(generator=g, dtype=torch.float32)


def pow_abs_sqrt_mean(case: dict, seed: int) -> dict:
    """tasks/pow_abs_sqrt_mean/reference.py:12-19 (U[0, scale) twice);
    baseline: N(0,1) twice, in the same order."""
    g = _gen(seed)
    shape = (case["batch_size"], 4, case["height"], case["width"])
    if case.get("kind") == "baseline":
        inp = torch.randn(shape, **_f(g))
        target = torch.randn(shape, **_f(g))
    else:
        scale = float(case.get("scale", 1.0))
        inp = torch.rand(shape, **_f(g)) * scale
        target = torch.rand(shape, **_f(g)) * scale
    return {"inp": inp, "target": target, "batch_size": case["batch_size"],
            "height": case["height"], "width": case["width"]}


def leaky(case: dict, seed: int) -> dict:
    """tasks/leaky/reference.py:12-23; baseline: x ~ 0.5 N + 0.3, mem0 = 0, beta = 0.9 and
    threshold = 1.0 broadcast to length H."""
    g = _gen(seed)
    T, B, H = case["T"], case["B"], case["H"]
    if case.get("kind") == "baseline":
        x = torch.randn(T, B, H, **_f(g)) * 0.5 + 0.3
        mem0 = torch.zeros(B, H)
        beta = torch.full((H,), 0.9)
        threshold = torch.full((H,), 1.0)
    else:
        x = torch.randn(T, B, H, **_f(g)) * 0.35 + 0.12
        std = float(case.get("mem0_std", 0.0))
        mem0 = torch.randn(B, H, **_f(g)) * std if std else torch.zeros(B, H)
        lo, hi = case.get("beta_range", [0.65, 0.98])
        beta = torch.rand(H, **_f(g)) * (hi - lo) + lo
        threshold = torch.rand(H, **_f(g)) * 0.6 + 0.8
    return {"input_current": x, "mem0": mem0, "beta": beta, "threshold": threshold,
            "T": T, "B": B, "H": H}


def reward_to_go(case: dict, seed: int) -> dict:
    """tasks/reward_to_go/reference.py:12-19 (reward U[0,1), done Bernoulli, last step
    done, gamma rounded to fp32); baseline: reward U[-1, 1)."""
    g = _gen(seed)
    B, T = case["B"], case["T"]
    reward = torch.rand(B, T, **_f(g))
    if case.get("kind") == "baseline":
        reward = reward * 2.0 - 1.0
    done = torch.rand(B, T, generator=g) < float(case["done_p"])
    done[:, -1] = True
    gamma = float(torch.tensor(case["gamma"], dtype=torch.float32))
    return {"reward": reward, "done": done, "gamma": gamma, "B": B, "T": T}


def ppo_clip(case: dict, seed: int) -> dict:
    """tasks/ppo_clip/reference.py:14-24; baseline: old ~ 0.5 N - 1, delta std 0.1, plus
    entropy ~ U[0, 2) and entropy_coef."""
    g = _gen(seed)
    shape = (case["B"], case["T"], case["H"])
    baseline = case.get("kind") == "baseline"
    old = torch.randn(shape, **_f(g)) * 0.5
    if baseline:
        old = old - 1.0
    std = 0.1 if baseline else float(case.get("delta_std", 0.12))
    delta = (torch.randn(shape, **_f(g)) * std).clamp(-20.0, 20.0)
    cur = old + delta
    adv = torch.randn(shape, **_f(g))
    out = {"B": case["B"], "T": case["T"], "H": case["H"], "current_log_prob": cur,
           "old_log_prob": old, "advantage": adv,
           "clip_epsilon": float(case.get("clip_epsilon", 0.2))}
    if baseline:
        out["entropy"] = torch.rand(shape, **_f(g)) * 2.0
        out["entropy_coef"] = float(case.get("entropy_coef", 0.01))
    return out


def efficient_kan(case: dict, seed: int) -> dict:
    """tasks/efficient_kan/reference.py:15-30 (x, grid, base_weight, spline_weight,
    spline_scaler in that draw order); baseline: all three weights N(0, 0.02^2)."""
    g = _gen(seed)
    B, I, O = case["B"], case["I"], case["O"]
    G, K = case.get("grid_size", 8), case.get("spline_order", 3)
    xr = float(case.get("x_range", 1.0))
    x = (torch.rand(B, I, **_f(g)) * 2.0 - 1.0) * xr
    step = 2.0 / G
    knots = torch.arange(-K, G + K + 1, dtype=torch.float32)
    grid = (knots * step - 1.0).expand(I, -1).contiguous()
    if case.get("kind") == "baseline":
        base_weight = torch.randn(O, I, **_f(g)) * 0.02
        spline_weight = torch.randn(O, I, G + K, **_f(g)) * 0.02
        spline_scaler = torch.randn(O, I, **_f(g)) * 0.02
    else:
        bound = 1.0 / math.sqrt(I)
        base_weight = (torch.rand(O, I, **_f(g)) * 2.0 - 1.0) * bound
        spline_weight = torch.randn(O, I, G + K, **_f(g)) * 0.05
        spline_scaler = torch.randn(O, I, **_f(g)) * 0.1 + 1.0
    return {"x": x, "grid": grid, "base_weight": base_weight, "spline_weight": spline_weight,
            "spline_scaler": spline_scaler, "grid_size": G, "spline_order": K,
            "B": B, "I": I, "O": O}


def quantize_e4m3(x: torch.Tensor) -> tuple[torch.Tensor, float]:
    """Per-tensor max-abs e4m3 quantisation, scale rounded to fp32
    (tasks/fp8_linear/reference.py:15-18)."""
    scale = float(np.float32(E4M3_MAX / max(x.abs().max().item(), 1e-9)))
    return (x * scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn), scale


def fp8_linear(case: dict, seed: int) -> dict:
    """tasks/fp8_linear/reference.py:21-31; baseline: x ~ N(0,1) and w ~ 0.02 N rounded
    to bf16 before quantisation."""
    g = _gen(seed)
    M, K, N = case["M"], case["K"], case["N"]
    if case.get("kind") == "baseline":
        x = torch.randn(M, K, **_f(g)).to(torch.bfloat16).float()
        w = (torch.randn(N, K, **_f(g)) * 0.02).to(torch.bfloat16).float()
    else:
        x = torch.randn(M, K, **_f(g))
        w = torch.randn(N, K, **_f(g)) * (1.0 / K ** 0.5)
    bias = (torch.randn(N, **_f(g)) * 0.05).to(torch.bfloat16)
    x_fp8, scale_x = quantize_e4m3(x)
    w_fp8, scale_w = quantize_e4m3(w)
    return {"M": M, "K": K, "N": N, "x_fp8": x_fp8, "scale_x": scale_x, "w_fp8": w_fp8,
            "scale_w": scale_w, "bias": bias}


_MAKERS = {
    "pow_abs_sqrt_mean": pow_abs_sqrt_mean,
    "leaky": leaky,
    "reward_to_go": reward_to_go,
    "ppo_clip": ppo_clip,
    "efficient_kan": efficient_kan,
    "fp8_linear": fp8_linear,
}


def make_inputs(op: str, case: dict, seed: int | None = None) -> dict:
    """Inputs of `op` for `case` (seed defaults to the case's own)."""
    return _MAKERS[op](case, case["seed"] if seed is None else seed)
