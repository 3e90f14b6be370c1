"""Verdict rows and tables from grading logs, with no GPU (grader/ledger.py): the columns
of a passing kernel, the status of failing ones, build failures, and `regrade` replaying
the rules over stored logs.  The logs are built here from small case reports."""
import json

import pytest

from cob_amd.grader import ledger

STEADY = {"alloc": 0, "host_copy": 0, "device_sync": 0, "other_stream": 0, "stream_sync": 0, "launch": 1,
          "memset": 0, "device_copy": 0}


def _tallies(mismatched=0, unwritten=0):
    return {"out": {"elements": 8, "size_ok": True, "mismatched": mismatched, "unwritten": unwritten,
                    "worst": 0.0, "first": None}}


def _case(name, first=0, second=0, counts=None, state="finished"):
    counts = counts or [STEADY, STEADY, STEADY]
    return {"case": name, "state": state, "repeat_identical": True,
            "calls": [{"call": i + 1, "inputs": "ABA"[i], "strays": [], "hip_calls": dict(c)}
                      for i, c in enumerate(counts)],
            "checks": {"1": _tallies(first), "2": _tallies(second)}}


def _log(kernel, passes, timing=None, build_ok=True, tail=""):
    log = {"kernel": kernel, "task": "reward_to_go", "build": {"ok": build_ok, "tail": tail},
           "passes": passes, "wall_s": 2.0}
    if timing:
        log["timing"] = {"case": "B64_T1024", "median_ms": timing, "range": {"kernel": 0.01}}
    return log


def test_passing_kernel_columns():
    first_call = dict(STEADY, alloc=1, launch=2)
    log = _log("k", [[_case("a", counts=[first_call, STEADY, STEADY]), _case("b")]] * 2,
               timing={"kernel": 0.004, "eager": 0.8, "expert": 0.0032})
    row = ledger.verdict_row(log)
    assert (row["status"], row["label"], row["passes"]) == ("pass", None, ["pass", "pass"])
    assert (row["kernel_ms"], row["x_eager"], row["pct_expert"]) == (0.004, 200.0, 80.0)
    assert (row["allocs_per_call"], row["launches_per_call"]) == (1, 2)     # the most any call made
    assert row["repeat_identical"] is True


@pytest.mark.parametrize("log,status,label", [
    (_log("k", [[_case("a", first=2)]], timing={"kernel": 1.0, "eager": 2.0}), "fail", "wrong value"),
    (_log("k", [[_case("a", second=8)]]), "fail", "stale state"),
    (_log("k", [[_case("a")], [_case("a", first=8, )]]), "flip", "wrong value"),
    (_log("k", [[_case("a", state="timeout")]]), "timeout", "timeout"),
    (_log("k", [], build_ok=False, tail="shim.hip:2:42: error: no matching function for call to 'reference'"),
     "compile_error", "signature mismatch"),
    (_log("k", [], build_ok=False, tail="k.hip:10:3: error: expected ';' after expression"), "compile_error", None),
])
def test_failing_kernel_status(log, status, label):
    row = ledger.verdict_row(log)
    assert (row["status"], row["label"]) == (status, label)
    assert row["kernel_ms"] is None and row["x_eager"] is None   # timing columns only for a pass


def test_tables_and_regrade(tmp_path):
    good = _log("taskops_reward_to_go", [[_case("a"), _case("b")]], timing={"kernel": 0.5, "eager": 10.0})
    bad = _log("planted_wrong_value", [[_case("a", first=1)]], timing={"kernel": 0.4, "eager": 10.0})
    for log in (good, bad):
        (tmp_path / f"{log['kernel']}.json").write_text(json.dumps(log))
    (tmp_path / "env.json").write_text(json.dumps({"gpu": "MI355X"}))
    rows = {r["kernel"]: r for r in ledger.tables(tmp_path)}
    assert set(rows) == {"taskops_reward_to_go", "planted_wrong_value"}
    assert rows["taskops_reward_to_go"]["x_eager"] == 20.0
    assert (rows["planted_wrong_value"]["label"], rows["planted_wrong_value"]["where"]) == ("wrong value", "call 1: out")
    lines = (tmp_path / "table.md").read_text().splitlines()
    assert lines[0].startswith("| kernel | task | status | label | where |") and len(lines) == 4
    assert json.loads((tmp_path / "verdicts.json").read_text())["planted_wrong_value"]["status"] == "fail"

    # `table` keeps a stored verdict; `regrade` recomputes it from the records and stores it.
    path = tmp_path / "taskops_reward_to_go.json"
    log = json.loads(path.read_text())
    log["verdict"] = dict(ledger.verdict_row(log), status="fail", label="stale state")
    path.write_text(json.dumps(log))
    assert {r["kernel"]: r["status"] for r in ledger.tables(tmp_path)}["taskops_reward_to_go"] == "fail"
    assert {r["kernel"]: r["status"] for r in ledger.tables(tmp_path, recompute=True)}["taskops_reward_to_go"] == "pass"
    assert json.loads(path.read_text())["verdict"]["status"] == "pass"


def test_cli(tmp_path, capsys):
    (tmp_path / "k.json").write_text(json.dumps(_log("k", [[_case("a")]], timing={"kernel": 0.25, "eager": 0.5})))
    assert ledger.main(["regrade", str(tmp_path)]) == 0
    out = capsys.readouterr().out
    assert "| k | reward_to_go | pass |" in out and "| 0.25 | 2 |" in out


@pytest.mark.gpu
@pytest.mark.timeout(400)
def test_grade_driver_on_gpu(tmp_path):
    """tests/grade_gpu.py end to end on two ops: logs, verdict rows, the table and the
    proof record, the planted libraries graded after the drop-ins."""
    import subprocess
    import sys
    from pathlib import Path
    from cob_amd.grader.plants import KINDS
    print("\n[grade] reward_to_go, fp8_linear", flush=True)
    drv = Path(__file__).resolve().parent / "grade_gpu.py"
    r = subprocess.run([sys.executable, "-u", str(drv), str(tmp_path), "--ops", "reward_to_go,fp8_linear",
                        "--passes", "1"], capture_output=True, text=True, timeout=360)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-3000:])
    rows = json.loads((tmp_path / "verdicts.json").read_text())
    dropins = {k: v for k, v in rows.items() if k.startswith("taskops_")}
    assert {r["task"]: r["status"] for r in dropins.values()} == {"reward_to_go": "pass", "fp8_linear": "pass"}
    assert all(r["kernel_ms"] > 0 and r["x_eager"] > 1 and r["launches_per_call"] == 1 for r in dropins.values())
    assert len(rows) == 2 + 2 * len(KINDS)
    proof = json.loads((tmp_path / "proof.json").read_text())
    assert proof["summary"] == {"references_pass": 2, "references": 2,
                                "planted_as_expected": 2 * len(KINDS), "planted": 2 * len(KINDS)}, proof["planted"]
