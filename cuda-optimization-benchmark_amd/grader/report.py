"""Verdicts and tables from per-kernel grading logs, with no GPU: the reproducible
pass/fail and timing tables of graders/verdict.py:64-141.

    python cuda-optimization-benchmark_amd/grader/report.py regrade LOG_DIR
    python cuda-optimization-benchmark_amd/grader/report.py table LOG_DIR

A log is one JSON file per graded kernel:

    {"key": ..., "task": op, "compile": {"ok": bool, "log_tail": str},
     "passes": [{"cases": [case record, ...]}, ...],     # grader/harness.py check()
     "timing": {"case": ..., "median_ms": {"kernel": ms, "torch": ms, "expert": ms},
                "spread": {...}},                         # grader/harness.py timing()
     "seconds": wall time of the grading run}

`table` writes results.json, verdicts.json and table.md from the verdicts stored in the
logs (or computed when absent); `regrade` recomputes every verdict from the records first,
so a change to the rules can be replayed over old logs.
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parents[2]))
    import __graft_entry__
    __graft_entry__.load_package()
    from cob_amd.grader.verdict import verdict as passes_verdict
else:
    from .verdict import verdict as passes_verdict

RESERVED = ("results.json", "verdicts.json", "env.json")
COLUMNS = ["Kernel", "Task", "Status", "Label", "Failed case / check", "Kernel ms", "x PyTorch eager",
           "% of expert speed", "Identical repeat", "Allocs per call", "Launches per call"]


def kernel_verdict(log: dict) -> dict:
    """Verdict of one kernel's log: the pass/fail rules over its passes, then the columns.
    A failed build is `compile_error`.  Timing columns are filled for passing kernels only."""
    v = {"status": None, "label": None, "failed_case": None, "failed_check": None, "kernel_ms": None,
         "speedup_vs_torch": None, "pct_of_expert": None, "identical_repeat": None,
         "allocs_per_call": None, "launches_per_call": None, "passes": []}
    comp = log.get("compile") or {}
    if not comp.get("ok"):
        v["status"] = "compile_error"
        tail = comp.get("log_tail", "")
        v["label"] = "signature mismatch" if "reference" in tail and "shim" in tail else None
        return v
    passes = []
    for p in log.get("passes", []):
        cases = []
        for rec in p.get("cases", []):
            rec = dict(rec)
            rec.setdefault("name", rec.get("case"))
            cases.append(rec)
        passes.append(cases)
    pv = passes_verdict(passes)
    for k in ("status", "label", "failed_case", "failed_check", "identical_repeat", "passes"):
        v[k] = pv[k]
    recs = [r for cases in passes for r in cases if r.get("proc") == "ok"]
    counts = [c["count"] for r in recs for c in r.get("calls", []) if c.get("count")]
    if counts:
        v["allocs_per_call"] = max(c["alloc"] for c in counts)
        v["launches_per_call"] = max(c["launch"] for c in counts)
    med = (log.get("timing") or {}).get("median_ms") or {}
    if v["status"] == "pass" and med.get("kernel"):
        v["kernel_ms"] = med["kernel"]
        if med.get("torch"):
            v["speedup_vs_torch"] = round(med["torch"] / med["kernel"], 3)
        if med.get("expert"):
            v["pct_of_expert"] = round(100 * med["expert"] / med["kernel"], 1)
    return v


def _fmt(x) -> str:
    if x is None:
        return ""
    if isinstance(x, float):
        return f"{x:.4g}"
    return str(x)


def logs(log_dir: Path):
    for p in sorted(Path(log_dir).glob("*.json")):
        if p.name in RESERVED:
            continue
        log = json.loads(p.read_text())
        if "task" in log:
            yield p, log


def write_tables(log_dir, recompute: bool = False) -> list[dict]:
    """results.json (one row per kernel), verdicts.json (by key) and table.md."""
    log_dir = Path(log_dir)
    rows = []
    for p, log in logs(log_dir):
        v = kernel_verdict(log) if recompute or "verdict" not in log else log["verdict"]
        t = log.get("timing") or {}
        rows.append(dict(key=log.get("key", p.stem), task=log["task"], **v,
                         spread=(t.get("spread") or {}).get("kernel"), seconds=log.get("seconds")))
    (log_dir / "results.json").write_text(json.dumps(rows, indent=1))
    (log_dir / "verdicts.json").write_text(json.dumps({r["key"]: r for r in rows}, indent=1))
    lines = ["| " + " | ".join(COLUMNS) + " |", "|" + "---|" * len(COLUMNS)]
    for r in rows:
        failed = " ".join(x for x in (r["failed_case"], r["failed_check"]) if x)
        cells = [r["key"], r["task"], r["status"], r["label"], failed, r["kernel_ms"], r["speedup_vs_torch"],
                 r["pct_of_expert"], r["identical_repeat"], r["allocs_per_call"], r["launches_per_call"]]
        lines.append("| " + " | ".join(_fmt(c) for c in cells) + " |")
    (log_dir / "table.md").write_text("\n".join(lines) + "\n")
    return rows


def regrade(log_dir) -> list[dict]:
    """Recompute every log's verdict from its records, store it back, rewrite the tables."""
    for p, log in logs(Path(log_dir)):
        log["verdict"] = kernel_verdict(log)
        p.write_text(json.dumps(log, indent=1))
    return write_tables(log_dir, recompute=False)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("cmd", choices=["regrade", "table"])
    ap.add_argument("log_dir")
    a = ap.parse_args(argv)
    rows = regrade(a.log_dir) if a.cmd == "regrade" else write_tables(a.log_dir)
    print((Path(a.log_dir) / "table.md").read_text(), end="")
    return 0 if rows else 1


if __name__ == "__main__":
    sys.exit(main())
