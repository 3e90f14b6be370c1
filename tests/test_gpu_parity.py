"""Parity of the HIP kernels with the CPU oracle, through the C ABI and the drop-in shims.

- Every hidden and public case of every task runs the grader's three-call protocol on
  guarded device buffers (4 KiB guards, 0xFF-poisoned outputs, seed / seed+7919 / seed),
  and must pass with identical bits on the repeat call.
- Every BASELINE workload is compared with the oracle over its whole output (the two GEMMs
  in blocks of rows, so every row tile of every kernel is covered), and every BASELINE
  call is repeated on the same buffers and must give the same bits.
- Edge cases: empty inputs, unaligned pointers, a non-default stream.
Tolerances are the task tolerances (pow additionally at BASELINE's rel 1e-5; leaky
bit-exact).
"""
import numpy as np
import pytest
import torch

from cob_amd import capi, inputs, tasks
from cob_amd.grader.labels import kernel_status
from cob_amd.grader.protocol import run_case
from cob_amd.grader.tolerance import tally
from oracle import exact

pytestmark = pytest.mark.gpu

CASES = [(op, c) for op in tasks.OPS for c in tasks.all_cases(op)]


@pytest.mark.parametrize("op,case", CASES, ids=[f"{op}-{c['name']}" for op, c in CASES])
def test_three_call_protocol(lib, op, case):
    print(f"\n[parity] {op} {case['name']}", flush=True)
    report = run_case(op, case, exact.reference_exact)
    st = kernel_status([[report]])
    assert st["status"] == "pass", (st, report.get("checks"), report.get("calls"))
    assert report["repeat_identical"]


def _baseline(op, key=None):
    case = tasks.BASELINE[key or op]
    return inputs.make_inputs(op, case)


def test_baseline_pow(lib):
    print("\n[parity] baseline pow 2^26", flush=True)
    inp = _baseline("pow_abs_sqrt_mean")
    got = capi.run_op(lib, "pow_abs_sqrt_mean", inp)["output"].item()
    want = float(exact.pow_abs_sqrt_mean(inp)["output"])
    assert abs(got - want) <= 1e-5 * abs(want), (got, want)     # BASELINE's rel 1e-5


def test_baseline_reward_to_go(lib):
    print("\n[parity] baseline reward_to_go 4096x4096", flush=True)
    inp = _baseline("reward_to_go")
    got = capi.run_op(lib, "reward_to_go", inp)["output"]
    t = tally(got.cpu(), exact.reward_to_go(inp)["output"], tasks.load_task("reward_to_go")["tolerance"])
    print(f"[parity] worst error {t['worst']:.4f} of the tolerance", flush=True)
    # fp64 carries and fp32 lane-local steps: a margin, not just a pass.
    assert t["mismatched"] == 0 and t["worst"] < 0.25, t


def test_baseline_leaky_bit_exact(lib):
    print("\n[parity] baseline leaky T256 B64 H4096", flush=True)
    inp = _baseline("leaky")
    got = capi.run_op(lib, "leaky", inp)
    want = exact.leaky(inp)
    assert np.array_equal(got["spikes"].cpu().numpy(), want["spikes"])
    assert np.array_equal(got["final_mem"].cpu().numpy(), want["final_mem"])


def test_baseline_ppo_entropy(lib):
    print("\n[parity] baseline ppo_clip 2^24 + entropy", flush=True)
    inp = _baseline("ppo_clip")
    got = capi.run_op(lib, "ppo_clip", inp)["output"].cpu()
    want = exact.ppo_clip(inp)["output"]
    t = tally(got, want, tasks.load_task("ppo_clip")["tolerance"])
    assert t["mismatched"] == 0, (t, got.tolist(), want.tolist())
    six = capi.run_op(lib, "ppo_clip", inp, entropy=False)["output"][:6].cpu()
    assert torch.equal(six, got[:6])                 # both entry points share the pass


def _row_blocks(n, block):
    return [np.arange(lo, min(n, lo + block)) for lo in range(0, n, block)]


def test_baseline_efficient_kan_full(lib):
    """All 8192 x 1024 outputs against the fp64 oracle, computed in blocks of 1024 rows:
    every 128-row tile and every column tile, so the XCD tile order at the BASELINE tile
    count is covered everywhere."""
    print("\n[parity] baseline efficient_kan B8192 I1024 O1024 G5 (all rows)", flush=True)
    inp = _baseline("efficient_kan")
    got = capi.run_op(lib, "efficient_kan", inp)["out"].cpu().numpy()
    tol = tasks.load_task("efficient_kan")["tolerance"]
    worst = 0.0
    for rows in _row_blocks(inp["B"], 1024):
        t = tally(got[rows], exact.efficient_kan(inp, rows=rows)["out"], tol)
        assert t["mismatched"] == 0, (rows[0], t)
        worst = max(worst, t["worst"])
    print(f"[parity] worst error {worst:.4f} of the tolerance", flush=True)


# (B, I, O, grid_size, spline_order, x_range, knots).  Order 3 with at most 16 knots per
# feature runs the fused fp16x3 MFMA kernel (C = 4, 7, 8, 11, 12 cover both padded basis
# widths); the others run the row-wise fp32 kernel.  Ragged B, I and O exercise every tile
# tail; x_range > 1 puts inputs outside the knot span.  Knots: "uniform" (the task's grid:
# the kernel's direct interval lookup), "random" (sorted random knots: the knot count),
# "jitter" (uniform plus noise of 1e-4 h: still the direct lookup, which must agree with
# the exact bases of the jittered knots), "mixed" (even features the task's grid, odd ones
# jittered by 1e-4 h: the kernel then reads every row's per-interval cubics, and the even
# rows' come from the cardinal closed form) and "mixed_edge" (even features jittered by
# 4e-7 h, still within the 5e-7 h of the closed form, so its cubics meet knots that are
# not exactly uniform).
KAN_SHAPES = [
    (130, 45, 70, 5, 3, 1.5, "uniform"),
    (67, 33, 258, 9, 3, 1.0, "random"),
    (40, 20, 36, 8, 3, 2.0, "uniform"),
    (9, 30, 31, 1, 3, 1.0, "uniform"),
    (33, 17, 19, 10, 3, 1.0, "uniform"),
    (50, 40, 40, 4, 3, 1.3, "random"),
    (70, 64, 96, 5, 3, 1.2, "jitter"),
    (70, 64, 96, 5, 3, 1.2, "mixed"),
    (64, 96, 40, 8, 3, 1.0, "mixed_edge"),
    (21, 40, 50, 6, 2, 1.2, "random"),
    (16, 12, 8, 13, 1, 1.0, "uniform"),
    # Row-wise path with more batch rows than a grid's y dimension takes (65,536), and with
    # more than one launch's 2^23 rows.
    (70001, 3, 5, 4, 2, 1.0, "uniform"),
    ((1 << 23) + 5, 1, 3, 3, 2, 1.0, "uniform"),
    # Split-K (fewer output tiles than CUs): 64 tiles and 5 feature groups split 2+2+1;
    # 96 tiles, ragged O and 3 groups split 2+1.
    (4096, 160, 512, 8, 3, 1.0, "uniform"),
    (4096, 90, 600, 5, 3, 1.0, "random"),
    # More than 1024 features: the weight packing reads each column twice instead of
    # keeping one batch of runs in registers (both padded basis widths).
    (24, 1100, 40, 5, 3, 1.0, "uniform"),
    (20, 1030, 33, 10, 3, 1.0, "random"),
]


@pytest.mark.parametrize("shape", KAN_SHAPES, ids=[f"B{s[0]}_I{s[1]}_O{s[2]}_G{s[3]}_K{s[4]}_{s[6]}" for s in KAN_SHAPES])
def test_efficient_kan_shapes(lib, shape):
    B, I, O, G, K, xr, knots = shape
    print(f"\n[parity] efficient_kan {shape}", flush=True)
    case = dict(name="k", seed=900 + B, B=B, I=I, O=O, grid_size=G, spline_order=K, x_range=xr)
    inp = inputs.make_inputs("efficient_kan", case)
    g = torch.Generator().manual_seed(B)
    L = G + 2 * K + 1
    if knots == "random":
        inp["grid"] = torch.sort(torch.rand(I, L, generator=g) * 3.0 - 1.5, dim=1).values.contiguous()
    elif knots in ("jitter", "mixed", "mixed_edge"):
        h = (inp["grid"][0, 1] - inp["grid"][0, 0]).item()
        noise = (torch.rand(I, L, generator=g) * 2 - 1) * 1e-4 * h
        if knots == "mixed":
            noise[0::2] = 0.0
        elif knots == "mixed_edge":
            noise[0::2] *= 0.004
        inp["grid"] = (inp["grid"] + noise).contiguous()
    want = exact.efficient_kan(inp)["out"]
    for _ in range(2):
        got = capi.run_op(lib, "efficient_kan", inp)["out"].cpu().numpy()
        t = tally(got, want, tasks.load_task("efficient_kan")["tolerance"])
        assert t["mismatched"] == 0, t


# The fast path's limits at BASELINE width (I = O = 1024, 4096 bases per output), with the
# reference's weight distributions (Ws 0.05 N, scaler 1 + 0.1 N: the spline term
# dominates) and BASELINE's: knot rows jittered by 4.5e-7 h stay on the cardinal pieces
# (uniform to 5e-7 h), which then differ from the exact bases by about 1e-6 of a basis
# value; rows jittered by 9e-6 h take the table's exact per-interval cubics.
@pytest.mark.parametrize("jitter", [4.5e-7, 9e-6])
@pytest.mark.parametrize("weights", ["reference", "baseline"])
def test_efficient_kan_knot_jitter_full_width(lib, jitter, weights):
    print(f"\n[parity] efficient_kan B256 I1024 O1024 G5, knots jittered by {jitter:g} h, {weights} weights", flush=True)
    case = dict(name="kj", seed=4620, B=256, I=1024, O=1024, grid_size=5, spline_order=3, x_range=1.0)
    if weights == "baseline":
        case["kind"] = "baseline"
    inp = inputs.make_inputs("efficient_kan", case)
    h = (inp["grid"][0, 1] - inp["grid"][0, 0]).item()
    g = torch.Generator().manual_seed(4621)
    noise = (torch.rand(inp["grid"].shape, generator=g, dtype=torch.float64) * 2 - 1) * jitter * h
    inp["grid"] = (inp["grid"].double() + noise).float().contiguous()
    want = exact.efficient_kan(inp)["out"]
    got = capi.run_op(lib, "efficient_kan", inp)["out"].cpu().numpy()
    t = tally(got, want, tasks.load_task("efficient_kan")["tolerance"])
    print(f"[parity] worst error {t['worst']:.4f} of the tolerance", flush=True)
    assert t["mismatched"] == 0, t


def test_efficient_kan_spline_weights_past_2gib(lib):
    """Ws of more than 2 GiB (O = 4096, I = 16400, C = 8: 2.15e9 bytes) on the fast path,
    with split-K (16 output tiles).  The weight packing addresses each output column's row
    of Ws from the row's own start, so the last columns, whose rows lie past 2 GiB, must
    read their real weights.  Only those 16 columns carry nonzero spline weights, which
    keeps the fp64 check small: the base term over every column, the spline term over the
    last 16."""
    B, I, O, G, K = 8, 16400, 4096, 5, 3
    C = G + K
    print(f"\n[parity] efficient_kan B{B} I{I} O{O} G{G}: Ws of {O * I * C * 4} bytes", flush=True)
    g = torch.Generator().manual_seed(7400)
    x = torch.rand(B, I, generator=g) * 2.0 - 1.0
    grid = (torch.arange(-K, G + K + 1, dtype=torch.float32) * (2.0 / G) - 1.0).expand(I, -1).contiguous()
    wb = torch.randn(O, I, generator=g) * 0.02
    sc = torch.randn(O, I, generator=g) * 0.1 + 1.0
    ws = torch.zeros(O, I, C)
    ws[-16:] = torch.randn(16, I, C, generator=g) * 0.05
    assert ws.numel() * 4 > 2 ** 31
    inp = dict(x=x, grid=grid, base_weight=wb, spline_weight=ws, spline_scaler=sc, grid_size=G,
               spline_order=K, B=B, I=I, O=O)
    got = capi.run_op(lib, "efficient_kan", inp)["out"].cpu().numpy()
    xd = x.double().numpy()
    want = (xd / (1.0 + np.exp(-xd))) @ wb.double().numpy().T
    bases = exact.b_splines(xd, grid.double().numpy(), K)
    w16 = (ws[-16:].double() * sc[-16:].double()[:, :, None]).reshape(16, -1).numpy()
    want[:, -16:] += bases.reshape(B, -1) @ w16.T
    t = tally(got, want, tasks.load_task("efficient_kan")["tolerance"])
    print(f"[parity] worst error {t['worst']:.4f} of the tolerance", flush=True)
    assert t["mismatched"] == 0, t


# (M, K, N, output offset in bf16 elements).  K % 16 == 0 with 16-byte aligned operands
# runs the wide kernel: its three epilogues (N % 8 == 0 and a 16-byte aligned output; N % 4
# == 0 and 8-byte aligned; otherwise), M and N tile tails, K not a multiple of its 128-wide
# step.  Up to 128 tiles of 256x256 (half the 256 CUs) it runs in its 128x256-tile form
# (fp8_gemm_half): every wide shape below up to the reference's timed M=2048 K=1024 N=4096;
# the M=2200 shapes (9 x 16 tiles) run the 256x256 form with the same tails.  K % 16 != 0
# runs the tiled kernel; M <= 64 the skinny (flat loads through LDS when K % 16 == 0, loads
# in the MFMA layout otherwise).
FP8_SHAPES = [
    (2048, 1024, 4096, 0),
    (2200, 144, 4000, 0),
    (2200, 144, 4004, 4),
    (2200, 176, 3999, 0),
    (300, 192, 264, 0),
    (300, 192, 264, 4),
    (257, 48, 260, 0),
    (130, 16, 257, 0),
    (333, 1000, 300, 0),
    (65, 40, 33, 1),
    (64, 4096, 96, 0),
    # skinny, flat 16-byte path: one to four row blocks (K slices of 512, 256, 256 and 128
    # bytes), K past the last whole slice, N past the last 16-column block
    (16, 4096, 272, 0),
    (17, 528, 100, 0),
    (40, 2064, 64, 2),
    (33, 48, 20, 0),
    (1, 16, 1, 0),
    (49, 400, 130, 0),
    # more than 32 column blocks, not a multiple of 32 (63 and 38): the XCD-aware block order
    # covers the first 32 and the rest keep their index
    (16, 512, 1000, 0),
    # skinny with K % 16 != 0 (the register path)
    (5, 40, 7, 0),
    (9, 40, 600, 0),
]


@pytest.mark.parametrize("shape", FP8_SHAPES, ids=[f"M{s[0]}_K{s[1]}_N{s[2]}_off{s[3]}" for s in FP8_SHAPES])
def test_fp8_linear_shapes(lib, shape):
    M, K, N, off = shape
    print(f"\n[parity] fp8_linear {shape}", flush=True)
    inp = inputs.make_inputs("fp8_linear", dict(name="f", seed=700 + M + N, M=M, K=K, N=N))
    args = capi.device_args("fp8_linear", inp)
    buf = torch.full((M * N + off + 8,), float("nan"), dtype=torch.bfloat16, device="cuda")
    out = buf[off:off + M * N].view(M, N)
    args["output"] = out
    want = exact.fp8_linear(inp)["output"]
    for _ in range(2):
        capi.call(lib, "fp8_linear", args)
        torch.cuda.synchronize()
        t = tally(out.cpu(), want, tasks.load_task("fp8_linear")["tolerance"])
        assert t["mismatched"] == 0, t
    assert torch.isnan(buf[:off].float()).all() and torch.isnan(buf[off + M * N:].float()).all()


def test_fp8_linear_k0(lib):
    """K == 0: the product is empty, so every output row is the bias (the wide kernel's
    copies are all out of range and zero-fill)."""
    M, N = 70, 72
    print("\n[parity] fp8_linear K=0", flush=True)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(3)) * 0.05).to(torch.bfloat16)
    args = dict(M=M, K=0, N=N, x_fp8=torch.empty(M, 0, dtype=torch.uint8, device="cuda"), scale_x=1.0,
                w_fp8=torch.empty(N, 0, dtype=torch.uint8, device="cuda"), scale_w=1.0,
                bias=bias.cuda(), output=torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda"))
    capi.call(lib, "fp8_linear", args)
    torch.cuda.synchronize()
    assert torch.equal(args["output"].cpu(), bias.expand(M, N))


@pytest.mark.parametrize("key", ["fp8_linear", "fp8_linear_m16"])
def test_baseline_fp8_full(lib, key):
    """Every output of the BASELINE fp8_linear calls (M = 4096: all 16 x 16 tiles of
    256 x 256; M = 16: the weight-streaming kernel) against the fp64 oracle."""
    print(f"\n[parity] baseline {key} (all rows)", flush=True)
    inp = _baseline("fp8_linear", key)
    got = capi.run_op(lib, "fp8_linear", inp)["output"].cpu()
    tol = tasks.load_task("fp8_linear")["tolerance"]
    worst = 0.0
    for rows in _row_blocks(inp["M"], 1024):
        t = tally(got[rows], exact.fp8_linear(inp, rows=rows)["output"], tol)
        assert t["mismatched"] == 0, (rows[0], t)
        worst = max(worst, t["worst"])
    print(f"[parity] worst error {worst:.4f} of the tolerance", flush=True)


BASELINE_CALLS = [("pow_abs_sqrt_mean", "pow_abs_sqrt_mean", None), ("reward_to_go", "reward_to_go", None),
                  ("leaky", "leaky", None), ("ppo_clip", "ppo_clip", True), ("ppo_clip", "ppo_clip", False),
                  ("efficient_kan", "efficient_kan", None), ("fp8_linear", "fp8_linear", None),
                  ("fp8_linear", "fp8_linear_m16", None)]


@pytest.mark.parametrize("op,key,entropy", BASELINE_CALLS,
                         ids=[f"{k}{'' if e is None else ('+entropy' if e else '-dropin')}" for _, k, e in BASELINE_CALLS])
def test_baseline_repeat_bits(lib, op, key, entropy):
    """A BASELINE call repeated on the same input buffers, into an output poisoned again
    with 0xFF, gives the same bits (fixed reduction orders, no float atomics, no state
    carried between calls)."""
    print(f"\n[parity] baseline repeat {key} entropy={entropy}", flush=True)
    inp = _baseline(op, key)
    args = capi.device_args(op, inp)
    if op == "ppo_clip":
        entry = "ppo_clip_entropy" if entropy else "ppo_clip"
        if not entropy:
            args = {k: v for k, v in args.items() if k not in ("entropy", "entropy_coef")}
        outs = {"output": torch.empty(8 if entropy else 6, device="cuda")}
    else:
        entry = op
        outs = {n: torch.empty(shape, dtype=dt, device="cuda") for n, (shape, dt) in capi.output_shapes(op, inp).items()}
    seen = []
    for _ in range(2):
        for o in outs.values():
            o.reshape(-1).view(torch.uint8).fill_(0xFF)
        capi.call(lib, entry, dict(args, **outs))
        torch.cuda.synchronize()
        seen.append({n: o.clone() for n, o in outs.items()})
    for n in outs:
        a, b = (x[n].reshape(-1).view(torch.uint8) for x in seen)
        assert torch.equal(a, b), n
        assert not bool((seen[0][n].reshape(-1).view(torch.uint8) == 0xFF).all())   # it wrote something


def test_pow_empty_and_unaligned(lib):
    out = torch.full((1,), 7.0, device="cuda")
    e = torch.empty(0, device="cuda")
    capi.call(lib, "pow_abs_sqrt_mean", dict(inp=e, target=e, batch_size=0, height=3, width=5, output=out))
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
    # 4-byte offset pointers take the unaligned path
    case = dict(name="u", seed=77, batch_size=3, height=5, width=7)
    inp = inputs.make_inputs("pow_abs_sqrt_mean", case)
    n = inp["inp"].numel()
    a = torch.empty(n + 1, device="cuda")[1:]
    b = torch.empty(n + 1, device="cuda")[1:]
    a.copy_(inp["inp"].reshape(-1))
    b.copy_(inp["target"].reshape(-1))
    capi.call(lib, "pow_abs_sqrt_mean", dict(inp=a, target=b, batch_size=3, height=5, width=7, output=out))
    torch.cuda.synchronize()
    want = float(exact.pow_abs_sqrt_mean(inp)["output"])
    assert abs(out.item() - want) <= 1e-6 * want


def test_rtg_empty_writes_nothing(lib):
    out = torch.full((4,), 3.0, device="cuda")
    e = torch.empty(0, device="cuda")
    d = torch.empty(0, dtype=torch.bool, device="cuda")
    capi.call(lib, "reward_to_go", dict(reward=e, done=d, gamma=0.9, B=0, T=4, output=out))
    torch.cuda.synchronize()
    assert (out == 3.0).all()


def test_leaky_zero_steps(lib):
    case = dict(name="z", seed=4, T=0, B=3, H=10, mem0_std=0.5)
    inp = inputs.make_inputs("leaky", case)
    got = capi.run_op(lib, "leaky", inp)
    assert torch.equal(got["final_mem"].cpu(), inp["mem0"])


def test_non_default_stream(lib):
    case = dict(name="s", seed=12, B=9, T=600, gamma=0.97, done_p=0.03)
    inp = inputs.make_inputs("reward_to_go", case)
    args = capi.device_args("reward_to_go", inp)
    out = torch.full((9, 600), float("nan"), device="cuda")
    args["output"] = out
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        capi.call(lib, "reward_to_go", args)   # enqueued on torch's current stream, s
    s.synchronize()
    t = tally(out.cpu(), exact.reward_to_go(inp)["output"], tasks.load_task("reward_to_go")["tolerance"])
    assert t["mismatched"] == 0, t


# Grids of the single-launch reductions: one workgroup per 2048 elements for pow (256
# threads x 2 x f32x4) and per 4096 for ppo_clip (512 x 2 x f32x4), capped at 512 and 256.
# The sizes give grids of 1, fewer than the 16 arrival groups, uneven group sizes, and the
# caps; each runs twice back to back (the arrival counters must be left zero).
GRID_SIZES = [1, 2, 15, 16, 17, 31, 33, 100, 255, 256, 257, 511, 512, 600]


@pytest.mark.parametrize("grid", GRID_SIZES)
def test_grid_reduction_sizes(lib, grid):
    print(f"\n[parity] grid reduction grid={grid}", flush=True)
    n = grid * 2048 - 5
    case = dict(name="g", seed=1000 + grid, batch_size=1, height=1, width=n // 4)
    inp = inputs.make_inputs("pow_abs_sqrt_mean", case)
    want = float(exact.pow_abs_sqrt_mean(inp)["output"])
    args = capi.device_args("pow_abs_sqrt_mean", inp)
    outs = [torch.full((1,), float("nan"), device="cuda") for _ in range(2)]
    for o in outs:
        capi.call(lib, "pow_abs_sqrt_mean", dict(args, output=o))
    torch.cuda.synchronize()
    for o in outs:
        assert abs(o.item() - want) <= 1e-5 * want

    m = grid * 4096 - 3
    pcase = dict(name="g", seed=2000 + grid, B=1, T=m, H=1)
    pinp = inputs.make_inputs("ppo_clip", pcase)
    pwant = exact.ppo_clip(pinp)["output"]
    pargs = capi.device_args("ppo_clip", pinp)
    pouts = [torch.full((6,), float("nan"), device="cuda") for _ in range(2)]
    for o in pouts:
        capi.call(lib, "ppo_clip", dict(pargs, output=o))
    torch.cuda.synchronize()
    tol = tasks.load_task("ppo_clip")["tolerance"]
    for o in pouts:
        t = tally(o.cpu(), pwant, tol)
        assert t["mismatched"] == 0, t
    assert torch.equal(pouts[0], pouts[1])


# reward_to_go's launch shape follows the row length in chunks of 256 steps: 1, 2 or 4
# waves of one chunk, 4 waves of 2, or 4 waves of 4 (rows past 4096 steps take several
# segments).  T values on either side of each boundary; T % 4 != 0 takes the element path.
RTG_T = [1, 255, 256, 257, 511, 512, 513, 1023, 1024, 1025, 1500, 2048, 2049, 4095, 4096, 4097, 9000]


@pytest.mark.parametrize("T", [4, 5])
def test_reward_to_go_rows_past_one_launch(lib, T):
    """More rows than one launch takes (2^23, one workgroup per row): the rows go out in two
    launches, the second starting at row 2^23 (T = 4 on the vector path, T = 5 on the element
    path)."""
    B = (1 << 23) + 3
    print(f"\n[parity] reward_to_go B={B} T={T}", flush=True)
    case = dict(name="rows", seed=77 + T, B=B, T=T, gamma=0.97, done_p=0.1)
    inp = inputs.make_inputs("reward_to_go", case)
    want = exact.reward_to_go(inp)["output"]
    got = capi.run_op(lib, "reward_to_go", inp)["output"].cpu()
    t = tally(got, want, tasks.load_task("reward_to_go")["tolerance"])
    assert t["mismatched"] == 0 and t["unwritten"] == 0, t


@pytest.mark.parametrize("T", RTG_T)
def test_reward_to_go_lengths(lib, T):
    print(f"\n[parity] reward_to_go T={T}", flush=True)
    case = dict(name="t", seed=3000 + T, B=3, T=T, gamma=0.98, done_p=0.02)
    inp = inputs.make_inputs("reward_to_go", case)
    want = exact.reward_to_go(inp)["output"]
    for _ in range(2):
        got = capi.run_op(lib, "reward_to_go", inp)["output"].cpu()
        t = tally(got, want, tasks.load_task("reward_to_go")["tolerance"])
        assert t["mismatched"] == 0, t
