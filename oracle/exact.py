"""numpy restatements of each task's `reference_exact` (the correctness reference).

Inputs are the dicts made by the package's input generators (CPU torch tensors and
Python scalars, keyed by C argument names); outputs are numpy arrays keyed by output
name.  Arithmetic is fp64 except `leaky`, whose reference is the fp32 step loop itself
(the operation order is the spec), and `fp8_linear`, whose fp64 result is rounded once to
bf16 the way torch converts float64 to bfloat16 (through fp32, nearest-even each time).

`rows` (efficient_kan, fp8_linear) restricts the computation to a subset of output rows,
for spot checks at full BASELINE sizes.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import e4m3


def _np(t: torch.Tensor, dtype=np.float64) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.contiguous().numpy().astype(dtype, copy=False)


def pow_abs_sqrt_mean(inp: dict) -> dict:
    """tasks/pow_abs_sqrt_mean/reference.py:22-32: mean(sqrt(|a-b|^2 + 0.001*0.001)) in fp64."""
    a = _np(inp["inp"]).reshape(-1)
    b = _np(inp["target"]).reshape(-1)
    d = np.abs(a - b)
    v = np.sqrt(d * d + 0.001 * 0.001)
    out = v.mean() if v.size else float("nan")
    return {"output": np.array(out, dtype=np.float64)}


def leaky(inp: dict) -> dict:
    """tasks/leaky/reference.py:26-37 (reference_exact is the same fp32 loop, :40).
    Every numpy op below rounds once in fp32, like each eager torch op."""
    x = _np(inp["input_current"], np.float32)
    T, B, H = x.shape
    with np.errstate(invalid="ignore"):
        beta = np.clip(_np(inp["beta"], np.float32), np.float32(0.0), np.float32(1.0)).reshape(1, H)
    th = _np(inp["threshold"], np.float32).reshape(1, H)
    mem = _np(inp["mem0"], np.float32).copy()
    spikes = np.empty_like(x)
    for t in range(T):
        reset = (mem >= th).astype(np.float32)
        mem = (beta * mem + x[t]) - reset * th
        spikes[t] = (mem >= th).astype(np.float32)
    return {"spikes": spikes, "final_mem": mem}


def reward_to_go(inp: dict) -> dict:
    """tasks/reward_to_go/reference.py:34-42: fp64 backward loop
    nxt = r[t] + gamma * keep[t] * nxt."""
    r = _np(inp["reward"]).T.copy()  # [T, B] so each step reads a contiguous row
    keep = (~inp["done"]).numpy().T.astype(np.float64)
    g = float(inp["gamma"])
    out = np.empty_like(r)
    nxt = np.zeros(r.shape[1])
    for t in range(r.shape[0] - 1, -1, -1):
        nxt = r[t] + g * keep[t] * nxt
        out[t] = nxt
    return {"output": out.T.copy()}


def _logsumexp(v: np.ndarray) -> float:
    m = v.max()
    return float(m + np.log(np.exp(v - m).sum()))


def ppo_clip(inp: dict) -> dict:
    """tasks/ppo_clip/reference.py:27-45 in fp64 with eps rounded to fp32 first (:43).
    Inputs holding `entropy` (the BASELINE variant) add mean(entropy) and
    -entropy_coef * mean(entropy) as outputs 7 and 8."""
    eps = float(np.float32(inp["clip_epsilon"]))
    cur = _np(inp["current_log_prob"]).reshape(-1)
    old = _np(inp["old_log_prob"]).reshape(-1)
    adv = _np(inp["advantage"]).reshape(-1)
    lw = cur - old
    ratio = np.exp(lw)
    lwc = np.clip(lw, math.log1p(-eps), math.log1p(eps))
    gain = np.minimum(ratio * adv, np.exp(lwc) * adv)
    n = lw.size
    ess = math.exp(2.0 * _logsumexp(lw) - _logsumexp(2.0 * lw)) / n
    vals = [-gain.mean(), (lwc != lw).astype(np.float64).mean(), ((ratio - 1.0) - lw).mean(),
            ess, ratio.max(), ratio.mean()]
    if "entropy" in inp:
        me = _np(inp["entropy"]).mean()
        vals += [me, -float(np.float32(inp["entropy_coef"])) * me]
    return {"output": np.array(vals, dtype=np.float64)}


def b_splines(x: np.ndarray, grid: np.ndarray, order: int) -> np.ndarray:
    """tasks/efficient_kan/reference.py:33-39: Cox-de Boor from order-0 indicators,
    vectorised over [B, I]; returns [B, I, G + order]."""
    xe = x[:, :, None]
    bases = ((xe >= grid[:, :-1]) & (xe < grid[:, 1:])).astype(np.float64)
    for k in range(1, order + 1):
        left = (xe - grid[:, :-(k + 1)]) / (grid[:, k:-1] - grid[:, :-(k + 1)])
        right = (grid[:, k + 1:] - xe) / (grid[:, k + 1:] - grid[:, 1:-k])
        bases = left * bases[:, :, :-1] + right * bases[:, :, 1:]
    return bases


def efficient_kan(inp: dict, rows=None) -> dict:
    """tasks/efficient_kan/reference.py:42-57 in fp64:
    silu(x) @ Wb^T + bsplines(x).reshape(B, I*C) @ (Ws * scaler[..., None]).reshape(O, I*C)^T."""
    x = _np(inp["x"])
    if rows is not None:
        x = x[np.asarray(rows)]
    grid = _np(inp["grid"])
    wb = _np(inp["base_weight"])
    ws = _np(inp["spline_weight"])
    sc = _np(inp["spline_scaler"])
    bases = b_splines(x, grid, int(inp["spline_order"]))
    silu = x / (1.0 + np.exp(-x))
    w = (ws * sc[:, :, None]).reshape(wb.shape[0], -1)
    out = silu @ wb.T + bases.reshape(x.shape[0], -1) @ w.T
    return {"out": out}


def round_f64_to_bf16(v: np.ndarray) -> np.ndarray:
    """fp64 -> bf16 as torch converts it: nearest-even to fp32, then nearest-even to bf16
    (NaN stays NaN).  Returned as float64 holding the bf16 values exactly."""
    f = np.asarray(v, dtype=np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).astype(np.float64)
    out[nan] = np.nan
    return out


def fp8_linear(inp: dict, rows=None) -> dict:
    """tasks/fp8_linear/reference.py:34-45 in fp64: (x/sx) @ (w/sw)^T + bias, one
    rounding to bf16."""
    xr = inp["x_fp8"].view(torch.uint8).numpy()
    if rows is not None:
        xr = xr[np.asarray(rows)]
    x = e4m3.decode(xr) / float(inp["scale_x"])
    w = e4m3.decode(inp["w_fp8"].view(torch.uint8).numpy()) / float(inp["scale_w"])
    bias = _np(inp["bias"])
    return {"output": round_f64_to_bf16(x @ w.T + bias)}


_FNS = {
    "pow_abs_sqrt_mean": pow_abs_sqrt_mean,
    "leaky": leaky,
    "reward_to_go": reward_to_go,
    "ppo_clip": ppo_clip,
    "efficient_kan": efficient_kan,
    "fp8_linear": fp8_linear,
}


def reference_exact(op: str, inp: dict, **kw) -> dict:
    return _FNS[op](inp, **kw)
