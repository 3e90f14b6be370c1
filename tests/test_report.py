"""Verdict/regrade tables from grading logs without a GPU (grader/report.py;
graders/verdict.py:64-141): the per-kernel verdict with its timing and call columns,
results.json / verdicts.json / table.md, and regrade replaying the rules over stored logs."""
import json

import pytest

from cob_amd.grader import report

CLEAN = {"alloc": 0, "host_copy": 0, "device_sync": 0, "other_stream": 0, "stream_sync": 0, "launch": 1,
         "memset": 0, "device_copy": 0}


def _call(n, count=None, **kw):
    c = {"call": n, "guards_ok": {"x": True, "out": True}, "inputs_unchanged": {"x": True},
         "count": dict(count or CLEAN)}
    c.update(kw)
    return c


def _case(name, call1=0, call2=0, poison=0, calls=None, **kw):
    r = {"name": name, "proc": "ok", "finished": True,
         "calls": calls if calls is not None else [_call(1), _call(2), _call(3)],
         "identical_repeat": True,
         "compare": {"call1": {"out": {"n": 10, "bad": call1, "bad_poison": poison, "shape_ok": True}},
                     "call2": {"out": {"n": 10, "bad": call2, "shape_ok": True}}}}
    r.update(kw)
    return r


def _log(key, passes, timing=None, compile_ok=True, tail=""):
    log = {"key": key, "task": "leaky", "compile": {"ok": compile_ok, "log_tail": tail},
           "passes": [{"cases": cases} for cases in passes], "seconds": 1.5}
    if timing:
        log["timing"] = {"case": "T256", "median_ms": timing, "spread": {"kernel": 0.01}}
    return log


def test_passing_kernel_columns():
    first = dict(CLEAN, alloc=1, launch=2)
    log = _log("k", [[_case("a", calls=[_call(1, first), _call(2), _call(3)]), _case("b")]] * 2,
               timing={"kernel": 0.05, "torch": 1.5, "expert": 0.04})
    v = report.kernel_verdict(log)
    assert v["status"] == "pass" and v["label"] is None and v["passes"] == ["pass", "pass"]
    assert v["kernel_ms"] == 0.05 and v["speedup_vs_torch"] == 30.0 and v["pct_of_expert"] == 80.0
    assert v["allocs_per_call"] == 1 and v["launches_per_call"] == 2   # the max over calls
    assert v["identical_repeat"] is True


@pytest.mark.parametrize("log,status,label", [
    (_log("k", [[_case("a", call1=2)]], timing={"kernel": 1.0, "torch": 2.0}), "fail", "wrong value"),
    (_log("k", [[_case("a", call2=10)]]), "fail", "stale state"),
    (_log("k", [[_case("a")], [_case("a", call1=1)]]), "flip", "wrong value"),
    (_log("k", [[_case("a", proc="timeout")]]), "timeout", "timeout"),
    (_log("k", [[_case("a", proc="crash", calls=[])]]), "grader_error", None),
    (_log("k", [], compile_ok=False, tail="shim.hip: no matching function for call to 'reference'"),
     "compile_error", "signature mismatch"),
    (_log("k", [], compile_ok=False, tail="error: expected ';'"), "compile_error", None),
])
def test_failing_kernel_status(log, status, label):
    v = report.kernel_verdict(log)
    assert (v["status"], v["label"]) == (status, label)
    assert v["kernel_ms"] is None and v["speedup_vs_torch"] is None  # timing only for passing kernels


def test_tables_and_regrade(tmp_path):
    good = _log("taskops_leaky", [[_case("a"), _case("b")]], timing={"kernel": 0.5, "torch": 10.0})
    bad = _log("planted_wrong", [[_case("a", call1=1)]], timing={"kernel": 0.4, "torch": 10.0})
    for log in (good, bad):
        (tmp_path / f"{log['key']}.json").write_text(json.dumps(log))
    (tmp_path / "env.json").write_text(json.dumps({"gpu": "x"}))
    rows = report.write_tables(tmp_path)
    by = {r["key"]: r for r in rows}
    assert set(by) == {"taskops_leaky", "planted_wrong"}
    assert by["taskops_leaky"]["speedup_vs_torch"] == 20.0 and by["planted_wrong"]["label"] == "wrong value"
    table = (tmp_path / "table.md").read_text().splitlines()
    assert table[0].startswith("| Kernel | Task | Status") and len(table) == 4
    assert json.loads((tmp_path / "verdicts.json").read_text())["planted_wrong"]["status"] == "fail"

    # A stored verdict is used as is by `table`; `regrade` recomputes it from the records.
    log = json.loads((tmp_path / "taskops_leaky.json").read_text())
    log["verdict"] = dict(report.kernel_verdict(log), status="fail", label="stale state")
    (tmp_path / "taskops_leaky.json").write_text(json.dumps(log))
    assert {r["key"]: r["status"] for r in report.write_tables(tmp_path)}["taskops_leaky"] == "fail"
    assert {r["key"]: r["status"] for r in report.regrade(tmp_path)}["taskops_leaky"] == "pass"
    assert json.loads((tmp_path / "taskops_leaky.json").read_text())["verdict"]["status"] == "pass"


def test_cli_regrade(tmp_path, capsys):
    (tmp_path / "k.json").write_text(json.dumps(_log("k", [[_case("a")]], timing={"kernel": 0.2, "torch": 0.4})))
    assert report.main(["regrade", str(tmp_path)]) == 0
    out = capsys.readouterr().out
    assert "| k | leaky | pass |" in out and "| 2 |" in out


def test_regrade_committed_gpu_logs(tmp_path):
    """The logs of a GPU grading run (tests/grade_gpu.py, kept in tests/golden/grade_logs)
    regrade on the CPU to the table that run printed: every kernel passes with identical
    repeats, and the steady calls' counts are in the logs."""
    import shutil
    from pathlib import Path
    src = Path(__file__).resolve().parent / "golden" / "grade_logs"
    for p in src.glob("*.json"):
        shutil.copy(p, tmp_path / p.name)
    rows = report.regrade(tmp_path)
    assert sorted(r["task"] for r in rows) == sorted(["efficient_kan", "fp8_linear", "leaky", "pow_abs_sqrt_mean",
                                                      "ppo_clip", "reward_to_go"])
    assert all(r["status"] == "pass" and r["identical_repeat"] for r in rows)
    assert (tmp_path / "table.md").read_text() == (src / "table.md").read_text()
    for p in src.glob("taskops_*.json"):
        log = json.loads(p.read_text())
        assert len(log["passes"]) == 2 and log["timing"]["median_ms"]["torch"] > 0
        steady = [c["count"] for pv in log["passes"] for r in pv["cases"] for c in r["calls"][1:]]
        assert steady and all(c["alloc"] == 0 and c["host_copy"] == 0 and c["device_sync"] == 0 for c in steady)


@pytest.mark.gpu
@pytest.mark.timeout(400)
def test_grade_driver_on_gpu(tmp_path):
    """tests/grade_gpu.py end to end on two ops: logs, verdicts and the table."""
    import subprocess
    import sys
    from pathlib import Path
    print("\n[grade] reward_to_go, fp8_linear", flush=True)
    drv = Path(__file__).resolve().parent / "grade_gpu.py"
    r = subprocess.run([sys.executable, "-u", str(drv), str(tmp_path), "--ops", "reward_to_go,fp8_linear",
                        "--passes", "1"], capture_output=True, text=True, timeout=360)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-3000:])
    rows = json.loads((tmp_path / "results.json").read_text())
    assert {r["task"]: r["status"] for r in rows} == {"reward_to_go": "pass", "fp8_linear": "pass"}
    assert all(r["kernel_ms"] > 0 and r["speedup_vs_torch"] > 1 and r["launches_per_call"] == 1 for r in rows)
