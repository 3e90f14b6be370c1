"""Special inputs through the HIP kernels, checked against the oracle and, where one
exists, against a closed form of the op (the closed forms named for each op's oracle):

- reward_to_go: every step done, or gamma = 0 (out = reward, bit for bit); no done step
  with a constant reward (r (1 - g^(T-t)) / (1 - g)); gamma = 1 (suffix sums);
- ppo_clip: cur == old (ratio 1: loss = -mean(A), clip fraction 0, kl 0, ess 1, max and
  mean ratio 1); log-ratios of +-20 (clipping and the max ratio far from 1);
- leaky: a membrane that lands exactly on the threshold (bit-exact with the oracle);
- pow_abs_sqrt_mean: inp == target (every term sqrt(1e-6));
- efficient_kan: zero spline weights (silu(x) @ Wb^T only), zero base weights (spline
  term only), x outside the knot span (spline term zero);
- fp8_linear: zero x (out = bias), e4m3 NaN codes in x (their rows NaN), +-448 codes; on the
  skinny, wide and tiled kernels.
"""
import math

import numpy as np
import pytest
import torch

from cob_amd import capi, inputs, tasks
from cob_amd.grader.tolerance import tally
from oracle import exact

pytestmark = pytest.mark.gpu


def _public(op):
    return next(c for c in tasks.all_cases(op) if c["name"].startswith("public_"))


def _agree(op, got, want):
    t = tally(got, want, tasks.load_task(op)["tolerance"])
    assert t["mismatched"] == 0, t


# ---- reward_to_go -------------------------------------------------------------------------

def _rtg_inputs(B, T, gamma, seed):
    inp = inputs.make_inputs("reward_to_go", dict(name="s", seed=seed, B=B, T=T, gamma=gamma, done_p=0.05))
    inp["gamma"] = float(np.float32(gamma))
    return inp


@pytest.mark.parametrize("T", [1, 300, 4096])
def test_rtg_all_done_and_gamma_zero_copy_the_reward(lib, T):
    print(f"\n[special] reward_to_go all-done / gamma 0, T={T}", flush=True)
    inp = _rtg_inputs(3, T, 0.97, 4100 + T)
    inp["done"] = torch.ones_like(inp["done"])
    got = capi.run_op(lib, "reward_to_go", inp)["output"].cpu()
    assert torch.equal(got, inp["reward"])
    inp = _rtg_inputs(3, T, 0.0, 4200 + T)
    got = capi.run_op(lib, "reward_to_go", inp)["output"].cpu()
    assert torch.equal(got, inp["reward"])


@pytest.mark.parametrize("T", [37, 1024, 4099])
def test_rtg_constant_reward_closed_form(lib, T):
    print(f"\n[special] reward_to_go constant reward, no done, T={T}", flush=True)
    g, r = float(np.float32(0.99)), 0.5
    inp = _rtg_inputs(2, T, 0.99, 4300 + T)
    inp["reward"] = torch.full_like(inp["reward"], r)
    inp["done"] = torch.zeros_like(inp["done"])
    got = capi.run_op(lib, "reward_to_go", inp)["output"].cpu()
    want = exact.reward_to_go(inp)["output"]
    _agree("reward_to_go", got, want)
    closed = np.array([r * (1.0 - g ** (T - t)) / (1.0 - g) for t in range(T)])
    _agree("reward_to_go", got[0].numpy(), closed)


def test_rtg_gamma_one_suffix_sums(lib):
    print("\n[special] reward_to_go gamma 1, no done", flush=True)
    inp = _rtg_inputs(4, 2000, 1.0, 4400)
    inp["done"] = torch.zeros_like(inp["done"])
    got = capi.run_op(lib, "reward_to_go", inp)["output"].cpu()
    want = exact.reward_to_go(inp)["output"]
    _agree("reward_to_go", got, want)
    suffix = np.cumsum(inp["reward"].double().numpy()[:, ::-1], axis=1)[:, ::-1]
    _agree("reward_to_go", got.numpy(), suffix)


def test_rtg_gamma_one_signed_rewards_full_rows(lib):
    """gamma = 1, U[-1, 1] rewards, no done step, BASELINE row length: the case where the
    fp32 lane steps' and wave scan's rounding errors never decay along the row, and outputs
    cross zero (where the bound is atol alone).  The task's rule must hold everywhere."""
    print("\n[special] reward_to_go gamma 1, U[-1,1], no done, T=4096", flush=True)
    g = torch.Generator().manual_seed(4410)
    B, T = 256, 4096
    inp = {"reward": torch.rand(B, T, generator=g) * 2 - 1, "done": torch.zeros(B, T, dtype=torch.bool),
           "gamma": 1.0, "B": B, "T": T}
    got = capi.run_op(lib, "reward_to_go", inp)["output"].cpu()
    t = tally(got, exact.reward_to_go(inp)["output"], tasks.load_task("reward_to_go")["tolerance"])
    print(f"[special] worst error {t['worst']:.4f} of the tolerance", flush=True)
    assert t["mismatched"] == 0, t


# ---- ppo_clip -----------------------------------------------------------------------------

@pytest.mark.parametrize("n", [(7, 13, 3), (4096, 256, 1)])
def test_ppo_unchanged_policy(lib, n):
    B, T, H = n
    print(f"\n[special] ppo_clip cur == old, {n}", flush=True)
    inp = inputs.make_inputs("ppo_clip", dict(name="s", seed=4500 + B, B=B, T=T, H=H))
    inp["current_log_prob"] = inp["old_log_prob"].clone()
    got = capi.run_op(lib, "ppo_clip", inp)["output"].cpu().numpy()
    want = exact.ppo_clip(inp)["output"]
    _agree("ppo_clip", got, want)
    adv = inp["advantage"].double().numpy()
    _agree("ppo_clip", got, np.array([-adv.mean(), 0.0, 0.0, 1.0, 1.0, 1.0]))


def test_ppo_large_log_ratios(lib):
    print("\n[special] ppo_clip log-ratios of +-20", flush=True)
    inp = inputs.make_inputs("ppo_clip", dict(name="s", seed=4600, B=33, T=17, H=5))
    sign = torch.where(torch.arange(inp["old_log_prob"].numel()) % 3 == 0, 20.0, -20.0)
    inp["current_log_prob"] = (inp["old_log_prob"].reshape(-1) + sign).reshape(inp["old_log_prob"].shape)
    got = capi.run_op(lib, "ppo_clip", inp)["output"].cpu().numpy()
    _agree("ppo_clip", got, exact.ppo_clip(inp)["output"])
    assert got[4] > 1e8  # max ratio is exp(20)


# ---- leaky --------------------------------------------------------------------------------

def test_leaky_membrane_on_the_threshold(lib):
    print("\n[special] leaky membrane exactly at the threshold", flush=True)
    inp = inputs.make_inputs("leaky", dict(name="s", seed=4700, T=6, B=3, H=40))
    inp["threshold"] = torch.full_like(inp["threshold"], 1.0)
    inp["mem0"] = torch.zeros_like(inp["mem0"])
    x = torch.zeros_like(inp["input_current"])
    x[0] = 1.0      # step 0: mem = beta * 0 + 1 = 1.0, exactly the threshold
    x[2] = 0.25     # later steps land on fractions that are exact in fp32
    x[3] = 0.75
    inp["input_current"] = x
    got = capi.run_op(lib, "leaky", inp)
    want = exact.leaky(inp)
    for name in want:
        assert np.array_equal(got[name].cpu().numpy(), np.asarray(want[name], dtype=np.float32)), name


# ---- pow_abs_sqrt_mean --------------------------------------------------------------------

def test_pow_identical_inputs(lib):
    print("\n[special] pow_abs_sqrt_mean inp == target", flush=True)
    inp = inputs.make_inputs("pow_abs_sqrt_mean", dict(name="s", seed=4800, batch_size=3, height=50, width=70))
    inp["target"] = inp["inp"].clone()
    got = capi.run_op(lib, "pow_abs_sqrt_mean", inp)["output"].cpu().numpy()
    _agree("pow_abs_sqrt_mean", got, exact.pow_abs_sqrt_mean(inp)["output"])
    _agree("pow_abs_sqrt_mean", got, np.array(math.sqrt(1e-6)))


# ---- efficient_kan ------------------------------------------------------------------------

def _kan_inputs(seed):
    return inputs.make_inputs("efficient_kan", dict(name="s", seed=seed, B=70, I=45, O=60, grid_size=5,
                                                    spline_order=3))


def test_kan_zero_spline_weights(lib):
    print("\n[special] efficient_kan Ws = 0", flush=True)
    inp = _kan_inputs(4900)
    inp["spline_weight"] = torch.zeros_like(inp["spline_weight"])
    got = capi.run_op(lib, "efficient_kan", inp)["out"].cpu().numpy()
    _agree("efficient_kan", got, exact.efficient_kan(inp)["out"])
    x = inp["x"].double().numpy()
    silu = x / (1.0 + np.exp(-x))
    _agree("efficient_kan", got, silu @ inp["base_weight"].double().numpy().T)


def test_kan_zero_base_weights(lib):
    print("\n[special] efficient_kan Wb = 0", flush=True)
    inp = _kan_inputs(4910)
    inp["base_weight"] = torch.zeros_like(inp["base_weight"])
    got = capi.run_op(lib, "efficient_kan", inp)["out"].cpu().numpy()
    _agree("efficient_kan", got, exact.efficient_kan(inp)["out"])


def test_kan_inputs_outside_the_knots(lib):
    print("\n[special] efficient_kan x outside the knot span", flush=True)
    inp = _kan_inputs(4920)
    span = float(inp["grid"].abs().max())
    sign = torch.where(torch.rand(inp["x"].shape, generator=torch.Generator().manual_seed(4920)) < 0.5, -1.0, 1.0)
    inp["x"] = (sign * (span + 0.5 + inp["x"].abs())).contiguous()
    got = capi.run_op(lib, "efficient_kan", inp)["out"].cpu().numpy()
    _agree("efficient_kan", got, exact.efficient_kan(inp)["out"])
    x = inp["x"].double().numpy()
    _agree("efficient_kan", got, (x / (1.0 + np.exp(-x))) @ inp["base_weight"].double().numpy().T)


# ---- fp8_linear ---------------------------------------------------------------------------

FP8_KERNELS = [(16, 256, 96), (300, 256, 264), (130, 40, 70)]  # skinny, wide, tiled


def _fp8_inputs(M, K, N, seed):
    return inputs.make_inputs("fp8_linear", dict(name="s", seed=seed, M=M, K=K, N=N))


@pytest.mark.parametrize("shape", FP8_KERNELS, ids=["skinny", "wide", "tiled"])
def test_fp8_zero_x_gives_the_bias(lib, shape):
    M, K, N = shape
    print(f"\n[special] fp8_linear zero x {shape}", flush=True)
    inp = _fp8_inputs(M, K, N, 5000 + M)
    inp["x_fp8"] = torch.zeros(M, K, dtype=torch.uint8).view(torch.float8_e4m3fn)
    got = capi.run_op(lib, "fp8_linear", inp)["output"].cpu()
    assert torch.equal(got, inp["bias"].reshape(1, N).expand(M, N))


@pytest.mark.parametrize("shape", FP8_KERNELS, ids=["skinny", "wide", "tiled"])
def test_fp8_nan_and_extreme_codes(lib, shape):
    M, K, N = shape
    print(f"\n[special] fp8_linear NaN and +-448 codes {shape}", flush=True)
    inp = _fp8_inputs(M, K, N, 5100 + M)
    xb = inp["x_fp8"].view(torch.uint8).clone()
    xb[1, 3] = 0x7F                      # NaN: row 1 of the output is NaN
    xb[M - 1, K - 1] = 0xFF              # -NaN: the last row too
    xb[0, :] = 0x7E                      # +448 across row 0
    wb = inp["w_fp8"].view(torch.uint8).clone()
    wb[N // 2, :] = 0xFE                 # -448 across one weight row
    inp["x_fp8"] = xb.view(torch.float8_e4m3fn)
    inp["w_fp8"] = wb.view(torch.float8_e4m3fn)
    got = capi.run_op(lib, "fp8_linear", inp)["output"].cpu()
    want = exact.fp8_linear(inp)["output"]
    _agree("fp8_linear", got.float().numpy(), want)
    assert torch.isnan(got[1].float()).all() and torch.isnan(got[M - 1].float()).all()
    assert not torch.isnan(got[0].float()).any()
