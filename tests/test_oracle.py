"""Pins every function of oracle/ (CPU only).

Each check is chosen so that a plausible slip in the oracle (a dropped term, a wrong
sign, index or axis, `>` for `>=`, a transposed operand, a wrong rounding) fails it:
closed forms, invariants, brute-force scalar loops on tiny inputs, and independent
implementations (scipy's B-spline basis, torch's own float8 and bfloat16 casts).  The
last group checks that the fp32 eager restatement (the CPU baseline) sits inside each
task tolerance of the fp64 oracle, as the reference's own test does
(graders/tests/test_grade.py:43-63).
"""
import math

import numpy as np
import pytest
import torch

from cob_amd import inputs, tasks
from cob_amd.grader.tolerance import tally
from oracle import e4m3, eager, exact


# ---- e4m3 decode -------------------------------------------------------------------------

def test_e4m3_known_values():
    t = e4m3.TABLE
    assert t[0x00] == 0.0 and t[0x80] == 0.0
    assert t[0x01] == 2.0 ** -9          # smallest subnormal
    assert t[0x07] == 7 * 2.0 ** -9      # largest subnormal
    assert t[0x08] == 2.0 ** -6          # smallest normal
    assert t[0x38] == 1.0                # exponent 7 = bias
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert math.isnan(t[0x7F]) and math.isnan(t[0xFF])
    assert np.isnan(t).sum() == 2


def test_e4m3_matches_torch_cast():
    raw = torch.arange(256, dtype=torch.uint8)
    want = raw.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    got = e4m3.decode(raw.numpy())
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_bf16_rounding_matches_torch():
    g = torch.Generator().manual_seed(0)
    v = torch.randn(200000, generator=g, dtype=torch.float64) * torch.exp(torch.randn(200000, generator=g, dtype=torch.float64) * 4)
    # values on and next to bf16 ties, including the fp32 double-rounding corner
    ties = torch.tensor([1 + 2 ** -8, 1 + 2 ** -8 + 2 ** -40, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 3.0e38, float("nan")],
                        dtype=torch.float64)
    v = torch.cat([v, ties])
    want = v.to(torch.bfloat16).to(torch.float64).numpy()
    got = exact.round_f64_to_bf16(v.numpy())
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()


# ---- pow_abs_sqrt_mean --------------------------------------------------------------------

def _pow_inp(a, b):
    a = torch.tensor(a, dtype=torch.float32).reshape(1, 4, 1, -1)
    b = torch.tensor(b, dtype=torch.float32).reshape(1, 4, 1, -1)
    return {"inp": a, "target": b, "batch_size": 1, "height": 1, "width": a.shape[-1]}


def test_pow_closed_forms():
    same = exact.pow_abs_sqrt_mean(_pow_inp([0.5] * 8, [0.5] * 8))["output"]
    assert same == pytest.approx(0.001, rel=1e-12)
    d = exact.pow_abs_sqrt_mean(_pow_inp([3.0] * 4, [-1.0] * 4))["output"]
    assert d == pytest.approx(math.sqrt(16.0 + 1e-6), rel=1e-14)
    mixed = exact.pow_abs_sqrt_mean(_pow_inp([1.0, 2.0, 0.0, 0.0], [0.0, 0.0, 0.0, 5.0]))["output"]
    want = (math.sqrt(1 + 1e-6) + math.sqrt(4 + 1e-6) + 0.001 + math.sqrt(25 + 1e-6)) / 4
    assert mixed == pytest.approx(want, rel=1e-14)


def test_pow_brute_force_small_case():
    case = tasks.all_cases("pow_abs_sqrt_mean")[0]
    inp = inputs.make_inputs("pow_abs_sqrt_mean", case)
    a = inp["inp"].reshape(-1).tolist()
    b = inp["target"].reshape(-1).tolist()
    want = sum(math.sqrt(abs(x - y) ** 2 + 1e-6) for x, y in zip(a, b)) / len(a)
    assert exact.pow_abs_sqrt_mean(inp)["output"] == pytest.approx(want, rel=1e-13)


def test_pow_baseline_expectation():
    # E sqrt(d^2 + 1e-6) for d ~ N(0, 2) is ~ 2/sqrt(pi) = 1.1284
    g = torch.Generator().manual_seed(7)
    a, b = torch.randn(1, 4, 256, 256, generator=g), torch.randn(1, 4, 256, 256, generator=g)
    v = exact.pow_abs_sqrt_mean({"inp": a, "target": b})["output"]
    assert v == pytest.approx(2 / math.sqrt(math.pi), rel=5e-3)


# ---- leaky ---------------------------------------------------------------------------------

def _leaky_inp(x, mem0, beta, th):
    x = torch.tensor(x, dtype=torch.float32)
    return {"input_current": x, "mem0": torch.tensor(mem0, dtype=torch.float32),
            "beta": torch.tensor(beta, dtype=torch.float32),
            "threshold": torch.tensor(th, dtype=torch.float32),
            "T": x.shape[0], "B": x.shape[1], "H": x.shape[2]}


def test_leaky_t1_closed_form_and_reset():
    # H=3 neurons: below threshold, exactly at threshold (a tie spikes: >=), reset case.
    x = [[[0.25, 1.0, 0.5]]]
    mem0 = [[0.5, 0.0, 1.5]]
    out = exact.leaky(_leaky_inp(x, mem0, [0.5, 0.0, 0.8], [1.0, 1.0, 1.2]))
    m = out["final_mem"][0]
    f = np.float32
    assert m[0] == f(f(0.5) * f(0.5)) + f(0.25)               # 0.5 -> 0.5
    assert m[1] == f(1.0)                                      # tie at the threshold
    assert m[2] == f(f(f(0.8) * f(1.5)) + f(0.5)) - f(1.2)     # mem0 >= th: subtract th
    assert out["spikes"][0, 0].tolist() == [0.0, 1.0, 0.0]


def test_leaky_beta_clamp_and_zero_input():
    x = np.zeros((5, 2, 3), dtype=np.float32)
    out = exact.leaky(_leaky_inp(x, np.zeros((2, 3)), [-0.5, 1.5, 0.3], [1.0, 1.0, 1.0]))
    assert not out["spikes"].any() and not out["final_mem"].any()
    # beta 1.5 clamps to 1: a constant input integrates linearly until the threshold.
    x = np.full((4, 1, 2), 0.25, dtype=np.float32)
    out = exact.leaky(_leaky_inp(x, np.zeros((1, 2)), [1.5, -3.0], [10.0, 10.0]))
    assert out["final_mem"].tolist() == [[1.0, 0.25]]


def test_leaky_matches_scalar_loop():
    case = dict(name="t", seed=9, T=12, B=3, H=7, mem0_std=0.3, beta_range=[-0.2, 1.2])
    inp = inputs.make_inputs("leaky", case)
    out = exact.leaky(inp)
    x = inp["input_current"].numpy()
    f = np.float32
    for b in range(3):
        for h in range(7):
            beta = min(max(float(inp["beta"][h]), 0.0), 1.0)
            th = f(inp["threshold"][h])
            m = f(inp["mem0"][b, h])
            for t in range(12):
                r = f(1.0) if m >= th else f(0.0)
                m = f(f(f(beta) * m) + x[t, b, h]) - f(r * th)
                assert out["spikes"][t, b, h] == (1.0 if m >= th else 0.0)
            assert out["final_mem"][b, h] == m


# ---- reward_to_go --------------------------------------------------------------------------

def _rtg_inp(r, d, g):
    r = torch.tensor(r, dtype=torch.float32)
    return {"reward": r, "done": torch.tensor(d, dtype=torch.bool), "gamma": g,
            "B": r.shape[0], "T": r.shape[1]}


def test_rtg_special_cases():
    r = [[0.5, -1.0, 2.0, 0.25]]
    assert np.array_equal(exact.reward_to_go(_rtg_inp(r, [[True] * 4], 0.9))["output"],
                          np.array(r, dtype=np.float32).astype(np.float64))
    assert exact.reward_to_go(_rtg_inp([[0.75], [-2.0]], [[False], [True]], 0.5))["output"].tolist() == [[0.75], [-2.0]]
    g, T = 0.97, 50
    out = exact.reward_to_go(_rtg_inp([[1.0] * T], [[False] * T], g))["output"][0]
    want = [(1 - g ** (T - t)) / (1 - g) for t in range(T)]
    assert np.allclose(out, want, rtol=1e-13)


def test_rtg_brute_force():
    case = dict(name="t", seed=5, B=4, T=37, gamma=0.9, done_p=0.2)
    inp = inputs.make_inputs("reward_to_go", case)
    out = exact.reward_to_go(inp)["output"]
    r = inp["reward"].double().numpy()
    d = inp["done"].numpy()
    g = inp["gamma"]
    for b in range(4):
        for t in range(37):
            s, w = 0.0, 1.0
            for k in range(t, 37):           # direct sum up to (and including) the next done
                s += w * r[b, k]
                if d[b, k]:
                    break
                w *= g
            assert out[b, t] == pytest.approx(s, rel=1e-12, abs=1e-12)


# ---- ppo_clip ------------------------------------------------------------------------------

def _ppo_inp(cur, old, adv, eps=0.2):
    t = lambda v: torch.tensor(v, dtype=torch.float32).reshape(1, -1, 1)
    return {"current_log_prob": t(cur), "old_log_prob": t(old), "advantage": t(adv),
            "clip_epsilon": eps, "B": 1, "T": len(cur), "H": 1}


def test_ppo_no_change():
    adv = [0.5, -1.0, 2.0, 0.25]
    out = exact.ppo_clip(_ppo_inp([0.1] * 4, [0.1] * 4, adv))["output"]
    assert out.tolist() == pytest.approx([-np.mean(adv), 0.0, 0.0, 1.0, 1.0, 1.0], abs=1e-15)


def test_ppo_hand_computed():
    eps = float(np.float32(0.2))
    lw = [0.5, -0.5, 0.1, 0.0]          # clipped high, clipped low, inside, inside
    adv = [1.0, -2.0, -1.0, 3.0]
    out = exact.ppo_clip(_ppo_inp(lw, [0.0] * 4, adv))["output"]
    lw32 = np.array(lw, dtype=np.float32).astype(np.float64)
    r = np.exp(lw32)
    gains = [(1 + eps) * 1.0, (1 - eps) * -2.0, r[2] * -1.0, r[3] * 3.0]  # min picks the clip
    assert out[0] == pytest.approx(-np.mean(gains), rel=1e-12)
    assert out[1] == 0.5
    assert out[2] == pytest.approx(np.mean((r - 1) - lw32), rel=1e-12)
    assert out[3] == pytest.approx(r.sum() ** 2 / (4 * (r * r).sum()), rel=1e-12)
    assert out[4] == pytest.approx(r.max(), rel=1e-15) and out[5] == pytest.approx(r.mean(), rel=1e-15)


def test_ppo_invariants_and_entropy():
    case = dict(tasks.BASELINE["ppo_clip"], B=64, T=32, H=1)
    inp = inputs.make_inputs("ppo_clip", case)
    out = exact.ppo_clip(inp)["output"]
    assert len(out) == 8
    assert 0 < out[3] <= 1 and out[4] >= out[5]
    me = inp["entropy"].double().mean().item()
    assert out[6] == pytest.approx(me, rel=1e-14)
    assert out[7] == pytest.approx(-float(np.float32(0.01)) * me, rel=1e-14)


# ---- efficient_kan -------------------------------------------------------------------------

def test_bsplines_match_scipy():
    from scipy.interpolate import BSpline
    G, K = 5, 3
    knots = np.arange(-K, G + K + 1) * (2.0 / G) - 1.0
    grid = np.tile(knots, (3, 1))
    x = np.linspace(-1.2, 1.2, 97).reshape(-1, 1).repeat(3, axis=1)
    got = exact.b_splines(x, grid, K)
    for c in range(G + K):
        want = BSpline.basis_element(knots[c:c + K + 2], extrapolate=False)(x[:, 0])
        want = np.nan_to_num(want)
        assert np.allclose(got[:, 0, c], want, atol=1e-14), c


def test_bsplines_partition_of_unity_and_support():
    G, K = 8, 3
    knots = np.arange(-K, G + K + 1) * (2.0 / G) - 1.0
    grid = knots[None, :]
    inside = np.linspace(-1.0, 0.999, 211)[:, None]
    s = exact.b_splines(inside, grid, K).sum(axis=-1)
    assert np.allclose(s, 1.0, atol=1e-14)
    outside = np.array([[-1.8], [1.9], [knots[-1] + 0.1]])
    assert not exact.b_splines(outside, grid, K).any()


def test_kan_terms_separately():
    case = dict(name="t", seed=3, B=6, I=5, O=4)
    inp = inputs.make_inputs("efficient_kan", case)
    x = inp["x"].double().numpy()
    silu = np.array([[v / (1 + math.exp(-v)) for v in row] for row in x])
    only_base = dict(inp, spline_weight=torch.zeros_like(inp["spline_weight"]))
    assert np.allclose(exact.efficient_kan(only_base)["out"], silu @ inp["base_weight"].double().numpy().T, rtol=1e-14)
    only_spline = dict(inp, base_weight=torch.zeros_like(inp["base_weight"]))
    bases = exact.b_splines(x, inp["grid"].double().numpy(), 3)
    ws = inp["spline_weight"].double().numpy() * inp["spline_scaler"].double().numpy()[:, :, None]
    want = np.einsum("bic,oic->bo", bases, ws)       # index-explicit, no reshape
    assert np.allclose(exact.efficient_kan(only_spline)["out"], want, rtol=1e-13)
    rows = [4, 1]
    assert np.array_equal(exact.efficient_kan(inp, rows=rows)["out"], exact.efficient_kan(inp)["out"][rows])


# ---- fp8_linear ----------------------------------------------------------------------------

def test_fp8_identity_and_zero():
    K = N = 16
    x = torch.zeros(3, K, dtype=torch.float32)
    x[0, 2], x[1, 5], x[2, 7] = 1.0, -2.0, 0.5
    w = torch.eye(N, K) * 448.0
    bias = (torch.arange(N, dtype=torch.float32) * 0.01).to(torch.bfloat16)
    inp = {"x_fp8": x.to(torch.float8_e4m3fn), "scale_x": 1.0, "w_fp8": w.to(torch.float8_e4m3fn),
           "scale_w": 448.0, "bias": bias, "M": 3, "K": K, "N": N}
    out = exact.fp8_linear(inp)["output"]
    want = bias.double().numpy()[None, :].repeat(3, 0)
    want[0, 2] += 1.0
    want[1, 5] -= 2.0
    want[2, 7] += 0.5
    assert np.array_equal(out, exact.round_f64_to_bf16(want))
    zero = dict(inp, x_fp8=torch.zeros(3, K).to(torch.float8_e4m3fn))
    assert np.array_equal(exact.fp8_linear(zero)["output"], bias.double().numpy()[None, :].repeat(3, 0))


def test_fp8_scales_divide_and_rows():
    case = dict(name="t", seed=8, M=7, K=32, N=9)
    inp = inputs.make_inputs("fp8_linear", case)
    x = e4m3.decode(inp["x_fp8"].view(torch.uint8).numpy())
    w = e4m3.decode(inp["w_fp8"].view(torch.uint8).numpy())
    raw = np.array([[sum(x[m, k] * w[n, k] for k in range(32)) for n in range(9)] for m in range(7)])
    want = raw / (inp["scale_x"] * inp["scale_w"]) + inp["bias"].double().numpy()
    got = exact.fp8_linear(inp)["output"]
    assert np.allclose(got, want, rtol=2 ** -7, atol=1e-6)
    assert np.array_equal(exact.fp8_linear(inp, rows=[3, 0])["output"], got[[3, 0]])


# ---- the eager fp32 baseline sits inside each tolerance of the fp64 oracle ------------------

@pytest.mark.parametrize("op", tasks.OPS)
def test_eager_within_tolerance_of_exact(op):
    task = tasks.load_task(op)
    case = next(c for c in task["cases"] if c.get("small"))
    inp = inputs.make_inputs(op, case)
    want = exact.reference_exact(op, inp)
    got = eager.reference(op, inp)
    for name in task["outputs"]:
        s = tally(got[name], want[name], task["tolerance"])
        assert s["mismatched"] == 0, (op, name, s)
