"""bench.py on the CPU: the algorithmic work each roofline divides by, derived here from the
BASELINE shapes (and the reference's timed fp8_linear case) by the byte and FLOP counts of each op's interface (not copied from the
table), the cache-cold rotation, and the refusals (more than one GPU, no GPU)."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402
from cob_amd import tasks  # noqa: E402

F32, BF16, BYTE = 4, 2, 1


def _work(key):
    """Bytes (HBM-bound) or FLOP (MFMA-bound) of one call at the BASELINE shape."""
    c = bench._case(bench.WORKLOADS[key][1])
    if key == "reward_to_go":                  # reward f32 + done bool in, f32 out
        return c["B"] * c["T"] * (F32 + BYTE + F32)
    if key == "pow_abs_sqrt_mean":             # two f32 inputs, one f32 scalar out
        return 2 * F32 * c["batch_size"] * 4 * c["height"] * c["width"] + F32
    if key == "leaky":                         # x in, spikes out per step; mem0 in, final out; beta, threshold
        return (c["T"] * c["B"] * c["H"] * 2 * F32 + c["B"] * c["H"] * 2 * F32 + c["H"] * 2 * F32)
    n = c.get("B", 0) * c.get("T", 0) * c.get("H", 0)
    if key == "ppo_clip":                      # cur, old, adv, entropy in; 8 f32 out
        return 4 * F32 * n + 8 * F32
    if key == "ppo_clip_dropin":               # cur, old, adv in; 6 f32 out
        return 3 * F32 * n + 6 * F32
    if key == "efficient_kan":                 # one contraction over I*(1 + G + K) per output
        return 2 * c["B"] * c["O"] * c["I"] * (1 + c["grid_size"] + c["spline_order"])
    if key in ("fp8_linear", "fp8_linear_timed"):
        return 2 * c["M"] * c["N"] * c["K"]
    if key == "fp8_linear_m16":                # w and x e4m3, bias bf16 in; bf16 out
        return c["N"] * c["K"] * BYTE + c["M"] * c["K"] * BYTE + c["N"] * BF16 + c["M"] * c["N"] * BF16
    if key == "quantize_e4m3":                 # fp32 x in, e4m3 codes out (the scale is 4 bytes)
        return c["M"] * c["K"] * (F32 + BYTE)
    raise KeyError(key)


@pytest.mark.parametrize("key", bench.ORDER)
def test_algorithmic_work(key):
    assert bench.WORKLOADS[key][3] == _work(key)


def test_every_workload_is_benched_and_bounded():
    assert sorted(bench.ORDER) == sorted(bench.WORKLOADS)
    for key, (entry, bkey, bound, _, dtype, _) in bench.WORKLOADS.items():
        assert (bkey in tasks.BASELINE or bkey == f"timed:{entry}") and bound in ("hbm", "mfma")
        if bound == "mfma":
            assert dtype in bench.PEAK_TFLOPS


def test_cold_rotation_exceeds_the_mall():
    """Working sets under the 256 MiB MALL rotate through enough copies to exceed it twice."""
    rtg = 4096 * 4096 * 9
    assert bench._copies(rtg) == 4 and 4 * rtg >= 2 * bench.MALL_BYTES
    assert bench._copies(2 * bench.MALL_BYTES) == 1
    assert bench._copies(1) == 24


def test_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""


def test_needs_a_gpu():
    """Without a GPU bench.py exits non-zero and prints no result line (no CPU fallback)."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--no-cpu", "--ops", "reward_to_go"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 1 and "needs a GPU" in r.stderr and r.stdout == ""


@pytest.mark.gpu
@pytest.mark.timeout(300)
def test_json_line_on_gpu():
    """One short bench.py run: a single JSON line with the contract's fields, the roofline of
    the timed kernel and the CPU baseline."""
    import json
    print("\n[bench] reward_to_go --steps 5", flush=True)
    r = subprocess.run([sys.executable, "-u", str(ROOT / "bench.py"), "--ops", "reward_to_go", "--steps", "5",
                        "--warmup", "1"], capture_output=True, text=True, timeout=280)
    assert r.returncode == 0, r.stderr[-3000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1
    d = json.loads(lines[0])
    assert d["n_gpus"] == 1 and d["steps"] == 5 and d["warmup"] == 1 and d["unit"] == "us/call"
    assert d["higher_is_better"] is False and d["vs_baseline"] is None and d["data"].startswith("synthetic")
    assert d["value"] > 0 and abs(d["ms_per_step"] * 1e3 - d["value"]) < 1e-3 * d["value"] + 1e-3
    assert "reward_to_go" in d["config"]["workload"]
    roof = d["roofline"]
    assert roof["bound"] == "hbm" and roof["peak"] == bench.HBM_PEAK_GBS and roof["unit"] == "GB/s"
    assert abs(roof["achieved"] - _work("reward_to_go") / (d["value"] * 1e-6) / 1e9) < 0.01 * roof["achieved"]
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    cpu = d["cpu_baseline"]
    assert cpu["value"] > 0 and cpu["unit"] == "us/call" and cpu["cores"] >= 1 and cpu["kind"] == "port"


def test_profile_summaries_name_their_source():
    """traffic.json and mfma.json carry the figures bench.py copies into the roofline, with
    the profiles/ file and commit they came from; bench tags each copied figure with that."""
    for name in ("traffic.json", "mfma.json"):
        s = bench._profile_json(name)
        assert set(s) >= {"values", "source", "commit"}, name
        assert s["source"].startswith("profiles/") and (ROOT / s["source"]).exists()
        assert len(s["commit"]) >= 7
        note = bench._provenance(s, name)
        assert s["commit"] in note and "not measured by this run" in note
    t = bench._profile_json("traffic.json")
    assert set(t["values"]) <= set(bench.WORKLOADS)
    assert "efficient_kan" in t["call_values"]
    assert t["call_values"]["efficient_kan"] >= t["values"]["efficient_kan"]


def test_profiling_json_writer(tmp_path):
    """profiling.py's summary writer: the figures plus source and commit."""
    import json
    from types import SimpleNamespace
    from cob_amd import profiling
    out = tmp_path / "x.json"
    profiling._write_json(str(out), {"values": {"leaky": 1}}, SimpleNamespace(source="profiles/a.md", commit="abc1234"))
    assert json.loads(out.read_text()) == {"values": {"leaky": 1}, "source": "profiles/a.md", "commit": "abc1234"}


def test_profiling_counters_table(tmp_path, capsys):
    """profiling.py counters: per kernel, the mean over dispatches of a counter summed over
    its instances, for the kernels whose names contain --kernel."""
    import sqlite3
    from cob_amd import profiling
    db = sqlite3.connect(tmp_path / "p_results.db")
    db.execute("create table counters_collection (kernel_name text, dispatch_id int, counter_name text, value real)")
    rows = [("fp8_gemm_half<2>", 1, "SQ_X", 3.0), ("fp8_gemm_half<2>", 1, "SQ_X", 5.0),
            ("fp8_gemm_half<2>", 2, "SQ_X", 10.0), ("other", 3, "SQ_X", 99.0), ("fp8_gemm_half<2>", 1, "SQ_Y", 7.0)]
    db.executemany("insert into counters_collection values (?, ?, ?, ?)", rows)
    db.commit()
    db.close()
    assert profiling.main(["counters", str(tmp_path), "SQ_X", "--kernel", "fp8_gemm"]) == 0
    lines = [l for l in capsys.readouterr().out.splitlines() if l.startswith("| SQ_")]
    assert lines == ["| SQ_X | `fp8_gemm_half<2>` | 2 | 9 |"]


def test_profiling_mfma_table_clock(tmp_path, capsys):
    """profiling.py mfma: busy % = MFMA busy cycles over (GRBM_GUI_ACTIVE per XCD x SIMDs), and
    the clock = GRBM_GUI_ACTIVE per XCD over the same dispatch's duration.  Two dispatches,
    2000 cycles in 1000 ns (2 GHz) at 50 % busy and 3000 cycles in 2000 ns (1.5 GHz) at 25 %,
    the counter summed over the 8 XCDs' instances."""
    import sqlite3
    from cob_amd import profiling
    db = sqlite3.connect(tmp_path / "m_results.db")
    db.execute("create table counters_collection (kernel_name text, dispatch_id int, counter_name text, value real)")
    db.execute("create table kernels (name text, dispatch_id int, duration real)")
    k, simds = "kan_fused<8>", profiling.MI355X_SIMDS
    rows = []
    for disp, cycles, busy in ((1, 2000.0, 0.5), (2, 3000.0, 0.25)):
        rows += [(k, disp, "GRBM_GUI_ACTIVE", cycles)] * profiling.MI355X_XCDS
        rows.append((k, disp, "SQ_VALU_MFMA_BUSY_CYCLES", busy * cycles * simds))
        rows.append((k, disp, "SQ_INSTS_VALU_MFMA_MOPS_F16", 10.0))
    db.executemany("insert into counters_collection values (?, ?, ?, ?)", rows)
    db.executemany("insert into kernels values (?, ?, ?)", [(k, 1, 1000.0), (k, 2, 2000.0)])
    db.commit()
    db.close()
    u = profiling.mfma_util(str(tmp_path))
    assert set(u) == {k}
    assert abs(u[k]["busy_pct"] - 37.5) < 1e-9
    assert abs(u[k]["clock_ghz"] - 1.75) < 1e-9
    assert u[k]["f16_flop"] == 512.0 * 10.0 and u[k]["dispatches"] == 2
    profiling.print_mfma(u)
    line = [l for l in capsys.readouterr().out.splitlines() if l.startswith("| `kan")][0]
    assert line == "| `kan_fused<8>` | 2 | 37.5 | 1.75 | 5120 | 0 |"
