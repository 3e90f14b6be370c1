"""fp32 PyTorch-CPU restatements of each task's eager `reference` — the reported CPU
baseline (never a correctness reference).  Each follows the op sequence of the cited
reference lines, so its cost profile (temporaries, passes) is the reference's.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def pow_abs_sqrt_mean(inp: dict) -> dict:
    """tasks/pow_abs_sqrt_mean/reference.py:22-28."""
    diff = torch.pow(torch.abs(inp["inp"] - inp["target"]), 2) + (0.001 * 0.001)
    return {"output": torch.mean(torch.sqrt(diff))}


def leaky(inp: dict) -> dict:
    """tasks/leaky/reference.py:26-37."""
    x = inp["input_current"]
    T, B, H = x.shape
    beta = inp["beta"].clamp(0.0, 1.0).view(1, H)
    th = inp["threshold"].view(1, H)
    mem = inp["mem0"].clone()
    spikes = torch.empty_like(x)
    for t in range(T):
        reset = (mem >= th).to(x.dtype)
        mem = beta * mem + x[t] - reset * th
        spikes[t] = (mem >= th).to(x.dtype)
    return {"spikes": spikes, "final_mem": mem}


def reward_to_go(inp: dict) -> dict:
    """tasks/reward_to_go/reference.py:22-31: log-depth doubling affine scan."""
    a = torch.where(inp["done"], 0.0, inp["gamma"]).to(torch.float32)
    b = inp["reward"].clone()
    T, d = b.shape[1], 1
    while d < T:
        b = torch.cat([b[:, :-d] + a[:, :-d] * b[:, d:], b[:, -d:]], dim=1)
        a = torch.cat([a[:, :-d] * a[:, d:], a[:, -d:] * 0.0], dim=1)
        d *= 2
    return {"output": b}


def ppo_clip(inp: dict) -> dict:
    """tasks/ppo_clip/reference.py:27-39 (+ the entropy terms for the BASELINE variant)."""
    cur, old, adv, eps = (inp["current_log_prob"], inp["old_log_prob"], inp["advantage"],
                          inp["clip_epsilon"])
    lw = cur - old
    ratio = torch.exp(lw)
    lwc = lw.clamp(math.log1p(-eps), math.log1p(eps))
    gain = torch.minimum(ratio * adv, torch.exp(lwc) * adv)
    flat = lw.reshape(-1)
    ess = torch.exp(2.0 * flat.logsumexp(0) - (2.0 * flat).logsumexp(0)) / flat.numel()
    vals = [-gain.mean(), (lwc != lw).to(lw.dtype).mean(), ((ratio - 1.0) - lw).mean(),
            ess, ratio.max(), ratio.mean()]
    if "entropy" in inp:
        me = inp["entropy"].mean()
        vals += [me, -inp["entropy_coef"] * me]
    return {"output": torch.stack(vals)}


def _b_splines(x, grid, order):
    xe = x.unsqueeze(-1)
    bases = ((xe >= grid[:, :-1]) & (xe < grid[:, 1:])).to(x.dtype)
    for k in range(1, order + 1):
        bases = ((xe - grid[:, :-(k + 1)]) / (grid[:, k:-1] - grid[:, :-(k + 1)])) * bases[:, :, :-1] + \
                ((grid[:, k + 1:] - xe) / (grid[:, k + 1:] - grid[:, 1:-k])) * bases[:, :, 1:]
    return bases.contiguous()


def efficient_kan(inp: dict) -> dict:
    """tasks/efficient_kan/reference.py:33-51."""
    x, wb = inp["x"], inp["base_weight"]
    bases = _b_splines(x, inp["grid"], inp["spline_order"])
    base_out = F.linear(F.silu(x), wb)
    w = (inp["spline_weight"] * inp["spline_scaler"].unsqueeze(-1)).reshape(wb.shape[0], -1)
    return {"out": base_out + F.linear(bases.reshape(x.shape[0], -1), w)}


def fp8_linear(inp: dict) -> dict:
    """tasks/fp8_linear/reference.py:34-41 in fp32."""
    x = inp["x_fp8"].to(torch.float32) / inp["scale_x"]
    w = inp["w_fp8"].to(torch.float32) / inp["scale_w"]
    return {"output": (x @ w.t() + inp["bias"].to(torch.float32)).to(torch.bfloat16)}


def quantize_e4m3(inp: dict) -> dict:
    """tasks/fp8_linear/reference.py:15-18 (`_quantize`): max |x|, fp32 scale, clamp, cast."""
    x = inp["x"]
    scale = float(torch.tensor(448.0 / max(x.abs().max().item(), 1e-9), dtype=torch.float32))
    return {"q": (x * scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), "scale": scale}


_FNS = {
    "pow_abs_sqrt_mean": pow_abs_sqrt_mean,
    "leaky": leaky,
    "reward_to_go": reward_to_go,
    "ppo_clip": ppo_clip,
    "efficient_kan": efficient_kan,
    "fp8_linear": fp8_linear,
    "quantize_e4m3": quantize_e4m3,
}


def reference(op: str, inp: dict) -> dict:
    return _FNS[op](inp)
