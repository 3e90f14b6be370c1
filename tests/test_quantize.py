"""Per-tensor e4m3 quantisation (tasks/fp8_linear/reference.py:15-18): the oracle, pinned,
and the HIP path (taskops_quantize_e4m3) against it, bit for bit.

The oracle's encode() is pinned against torch's float8_e4m3fn cast on every e4m3 value,
every midpoint between neighbours and the fp32 values either side of it, signed zeros,
signed NaN and random values; quantize() is pinned against cob_amd.inputs.quantize_e4m3,
whose output the golden input digests pin to the reference's own `_quantize`.  Bytes
must match exactly except NaN results, where 0x7F and 0xFF both count (e4m3.same_codes).
"""
import numpy as np
import pytest
import torch

from cob_amd import capi, inputs
from oracle import e4m3


def _special_values() -> np.ndarray:
    pos = e4m3.TABLE[:0x7F]
    vals = []
    for i in range(len(pos)):
        vals.append(pos[i])
        if i + 1 < len(pos):
            mid = np.float32((pos[i] + pos[i + 1]) / 2)
            vals += [mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(1000))]
    v = np.array(vals, dtype=np.float32)
    return np.concatenate([v, -v, np.array([0.0, -0.0, 1e-30, -1e-30, 448.0, -448.0], np.float32)])


def test_encode_matches_torch_cast():
    rng = np.random.default_rng(0)
    v = np.concatenate([_special_values(), np.array([np.nan, -np.nan], np.float32),
                        rng.uniform(-448, 448, 100_000).astype(np.float32),
                        (rng.standard_normal(100_000) * 0.01).astype(np.float32)])
    want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(e4m3.encode(v), want)


def test_encode_decode_round_trip():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    assert np.array_equal(e4m3.encode(e4m3.decode(codes)), codes)


@pytest.mark.parametrize("kind", ["normal", "wide", "zeros", "one", "nan", "inf", "tiny"])
def test_quantize_matches_pinned_inputs(kind):
    g = torch.Generator().manual_seed(11)
    x = {"normal": torch.randn(3001, generator=g),
         "wide": torch.randn(517, generator=g) * 1e4,
         "zeros": torch.zeros(64),
         "one": torch.tensor([-2.5]),
         "nan": torch.randn(100, generator=g).index_fill_(0, torch.tensor([37]), float("nan")),
         "inf": torch.randn(100, generator=g).index_fill_(0, torch.tensor([5]), float("inf")),
         "tiny": torch.randn(100, generator=g) * 1e-20}[kind]
    q_want, s_want = inputs.quantize_e4m3(x)
    q, s = e4m3.quantize(x.numpy())
    assert e4m3.same_codes(q, q_want.view(torch.uint8).numpy())
    assert (np.isnan(s) and np.isnan(s_want)) or np.float32(s) == np.float32(s_want)


def test_quantize_closed_forms():
    x = np.array([1.0, -3.0, 0.5], np.float32)
    q, s = e4m3.quantize(x)
    assert s == np.float32(448.0 / 3.0)
    assert q[1] == 0xFE                      # -amax maps to -448
    assert e4m3.decode(q)[0] == pytest.approx(448.0 / 3.0, rel=2 ** -3)


# -------------------------------------------------------------------------------------
# HIP path
# -------------------------------------------------------------------------------------

def _run_gpu(lib, x: torch.Tensor, q_off: int = 0, x_off: int = 0):
    n = x.numel()
    xb = torch.empty(n + x_off, dtype=torch.float32, device="cuda")
    xd = xb[x_off:]
    xd.copy_(x.reshape(-1))
    qb = torch.full((n + q_off + 64,), 0xA5, dtype=torch.uint8, device="cuda")
    qd = qb[q_off:q_off + n]
    sd = torch.full((1,), -7.0, device="cuda")
    capi.call(lib, "quantize_e4m3", dict(x=xd, n=n, q=qd, scale=sd))
    torch.cuda.synchronize()
    tail = qb[q_off + n:].cpu()
    assert (tail == 0xA5).all() and (qb[:q_off].cpu() == 0xA5).all(), "write outside q"
    return qd.cpu().numpy(), np.float32(sd.item())


# One workgroup of the fused path holds 16384 elements; tensors above its resident capacity
# (1024 workgroups on 256 CUs, 2^24 elements) and unaligned ones take the two-pass path.
@pytest.mark.gpu
@pytest.mark.parametrize(
    "n", [1, 15, 16, 17, 4095, 16384, 16385, 49151, 65537, 1 << 20, 1 << 24, (1 << 24) + 1, 24_000_001]
)
def test_gpu_quantize_sizes(lib, n):
    print(f"\n[parity] quantize_e4m3 n={n}", flush=True)
    x = torch.randn(n, generator=torch.Generator().manual_seed(n)) * 3.0
    q, s = _run_gpu(lib, x)
    q_want, s_want = e4m3.quantize(x.numpy())
    assert s == s_want
    assert np.array_equal(q, q_want)


def _random_quantize_cases(count=24, seed=20261203):
    """Seeded draws: size log-uniform over 1 .. 3M, x and q offsets (unaligned ones take the
    two-pass path), and the values' magnitude."""
    import random
    rng = random.Random(seed)
    return [(int(10 ** rng.uniform(0, 6.5)), rng.choice([0, 0, 1, 3]), rng.choice([0, 0, 1, 2, 3]),
             rng.choice([1e-6, 1.0, 7.0, 1e4])) for _ in range(count)]


@pytest.mark.gpu
@pytest.mark.parametrize("n,x_off,q_off,mag", _random_quantize_cases())
def test_gpu_quantize_random(lib, n, x_off, q_off, mag):
    """Random sizes, offsets and magnitudes: the codes and the scale equal the oracle's."""
    print(f"\n[parity] quantize_e4m3 random n={n} x_off={x_off} q_off={q_off} mag={mag}", flush=True)
    x = torch.randn(n, generator=torch.Generator().manual_seed(n + 17 * x_off + q_off)) * mag
    q, s = _run_gpu(lib, x, q_off=q_off, x_off=x_off)
    q_want, s_want = e4m3.quantize(x.numpy())
    assert s == s_want
    assert e4m3.same_codes(q, q_want)


@pytest.mark.gpu
def test_gpu_quantize_cast_table(lib):
    """Every e4m3 value, midpoint and neighbour with scale exactly 1 (|x| max = 448): the
    hardware conversion's rounding, signed zeros and subnormals."""
    x = torch.from_numpy(_special_values())
    q, s = _run_gpu(lib, x)
    assert s == np.float32(1.0)
    assert np.array_equal(q, e4m3.encode(x.numpy()))


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["nan", "zeros", "inf", "unaligned", "q_off4", "q_off2"])
def test_gpu_quantize_edges(lib, case):
    print(f"\n[parity] quantize_e4m3 {case}", flush=True)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(10_003, generator=g)
    q_off = x_off = 0
    if case == "nan":
        x[4321] = float("nan")
    elif case == "zeros":
        x = torch.zeros(4099)
    elif case == "inf":
        x[17] = float("-inf")
    elif case == "unaligned":
        q_off, x_off = 3, 1
    else:
        q_off = int(case[-1])
    q, s = _run_gpu(lib, x, q_off=q_off, x_off=x_off)
    q_want, s_want = e4m3.quantize(x.numpy())
    assert (np.isnan(s) and np.isnan(s_want)) or s == s_want
    assert e4m3.same_codes(q, q_want)


@pytest.mark.gpu
def test_gpu_quantize_baseline_operands(lib):
    """The fp8_linear BASELINE operands: quantising the bf16-rounded x on the GPU gives the
    bytes and scale the input builder makes on the CPU."""
    g = torch.Generator().manual_seed(404)
    x = torch.randn(4096, 4096, generator=g).to(torch.bfloat16).float()
    q, s = _run_gpu(lib, x)
    q_want, s_want = inputs.quantize_e4m3(x)
    assert s == np.float32(s_want)
    assert np.array_equal(q, q_want.view(torch.uint8).numpy().reshape(-1))


@pytest.mark.gpu
def test_gpu_quantize_empty_writes_nothing(lib):
    sd = torch.full((1,), -7.0, device="cuda")
    capi.call(lib, "quantize_e4m3", dict(x=torch.empty(0, device="cuda"), n=0,
                                         q=torch.empty(0, dtype=torch.uint8, device="cuda"), scale=sd))
    torch.cuda.synchronize()
    assert sd.item() == -7.0


@pytest.mark.gpu
def test_gpu_quantize_back_to_back(lib):
    """Calls queued without a host sync between them, a NaN tensor among them: the grid
    barrier's state must start clean each call (a NaN max left over would poison the next)."""
    g = torch.Generator().manual_seed(77)
    xs = [torch.randn(300_000, generator=g) * 2.0, torch.randn(300_000, generator=g),
          torch.randn(70_000, generator=g) * 50.0, torch.randn(5, generator=g)]
    xs[1][123] = float("nan")
    dev = [x.to("cuda") for x in xs]
    qs = [torch.empty(x.numel(), dtype=torch.uint8, device="cuda") for x in xs]
    ss = [torch.empty(1, device="cuda") for _ in xs]
    for _ in range(2):
        for x, q, s in zip(dev, qs, ss):
            capi.call(lib, "quantize_e4m3", dict(x=x, n=x.numel(), q=q, scale=s))
    torch.cuda.synchronize()
    for x, q, s in zip(xs, qs, ss):
        q_want, s_want = e4m3.quantize(x.numpy())
        got = np.float32(s.item())
        assert (np.isnan(got) and np.isnan(s_want)) or got == s_want
        assert e4m3.same_codes(q.cpu().numpy(), q_want)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 16385, 1 << 20])
def test_gpu_quantize_fallback_path_same_bits(lib, n):
    """The fused kernel's bounded wait, forced to time out at once (a test hook sets its poll
    count to 0): every workgroup finds the max itself, and the bits equal the barrier path's
    and the oracle's."""
    import ctypes
    print(f"\n[parity] quantize_e4m3 fallback n={n}", flush=True)
    x = torch.randn(n, generator=torch.Generator().manual_seed(n + 3)) * 7.0
    if n == 16385:
        x[n // 3] = float("nan")                # a NaN carries through either path
    q0, s0 = _run_gpu(lib, x)
    hook = lib.taskops_testing_quantize_spin_limit
    hook.argtypes = [ctypes.c_uint]
    hook(0)
    try:
        q1, s1 = _run_gpu(lib, x)
    finally:
        hook(1 << 14)
    q2, s2 = _run_gpu(lib, x)                 # and the barrier path again afterwards
    q_want, s_want = e4m3.quantize(x.numpy())
    for q, s in ((q0, s0), (q1, s1), (q2, s2)):
        assert (np.isnan(s) and np.isnan(s_want)) or s == s_want
        assert e4m3.same_codes(q, q_want)
    assert np.array_equal(q0, q1) and np.array_equal(q0, q2)


@pytest.mark.gpu
def test_gpu_quantize_graph_replay(lib):
    """Captured into a graph, the fused kernel's barrier state carries across replays (the
    parity word flips every launch, and each launch clears the other set of words)."""
    n = 300_000
    xd = torch.empty(n, device="cuda")
    q = torch.empty(n, dtype=torch.uint8, device="cuda")
    sd = torch.empty(1, device="cuda")
    args = dict(x=xd, n=n, q=q, scale=sd)
    xd.copy_(torch.randn(n, generator=torch.Generator().manual_seed(1)))
    capi.call(lib, "quantize_e4m3", args)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        capi.call(lib, "quantize_e4m3", args)
    for k in range(4):
        x = torch.randn(n, generator=torch.Generator().manual_seed(10 + k)) * (k + 1)
        xd.copy_(x)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        q_want, s_want = e4m3.quantize(x.numpy())
        assert float(sd.item()) == float(s_want)
        assert np.array_equal(q.cpu().numpy(), q_want)
