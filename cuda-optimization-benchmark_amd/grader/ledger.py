"""Grading logs → one verdict row per kernel → verdicts.json and table.md, with no GPU.

    python cuda-optimization-benchmark_amd/grader/ledger.py table   LOG_DIR
    python cuda-optimization-benchmark_amd/grader/ledger.py regrade LOG_DIR

A log is one JSON file per graded kernel, written by the grading driver:

    {"kernel": key, "task": op,
     "build":  {"ok": bool, "lib": file, "tail": last lines of the build log},
     "passes": [[case report, ...], ...],            # grader/protocol.py run_case
     "timing": {"case": name, "median_ms": {"kernel": ms, "eager": ms, "expert": ms},
                "range": {...}},                     # grader/protocol.py time_case
     "wall_s": seconds, "env": {...},
     "verdict": row}                                 # filled by this module

The columns are the reference's (graders/verdict.py:103-115 defines them): status and
label, where it failed, the kernel's ms per call, the speedup over PyTorch eager, the
percentage of the expert kernel's speed, whether call 3 repeated call 1's bits, and the
most allocations and launches any one call made.  `table` uses each log's stored verdict
(computing it when absent); `regrade` recomputes every verdict from the records first,
so changed rules can be replayed over old logs.
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
    from cob_amd.grader.labels import kernel_status
else:
    from .labels import kernel_status

OUTPUT_FILES = ("verdicts.json", "table.md", "env.json")
HEADER = ("kernel", "task", "status", "label", "where", "kernel ms", "× eager", "% of expert",
          "repeat bits", "allocs/call", "launches/call")
# Compiler messages that mean the shim's call of reference(...) did not fit the kernel's
# declaration, i.e. the kernel does not have the task's signature.
_MISMATCH = ("no matching function for call to 'reference'", "too many arguments to function",
             "too few arguments to function", "cannot initialize a parameter")


def _most(counts: list[dict], key: str):
    vals = [c.get(key) for c in counts if c.get(key) is not None]
    return max(vals) if vals else None


def verdict_row(log: dict) -> dict:
    """The verdict of one kernel's log."""
    row = {"kernel": log.get("kernel"), "task": log.get("task"), "status": None, "label": None,
           "where": None, "case": None, "kernel_ms": None, "x_eager": None, "pct_expert": None,
           "repeat_identical": None, "allocs_per_call": None, "launches_per_call": None, "passes": []}
    build = log.get("build") or {}
    if not build.get("ok"):
        tail = build.get("tail", "")
        row["status"] = "compile_error"
        row["label"] = "signature mismatch" if any(m in tail for m in _MISMATCH) else None
        return row
    st = kernel_status(log.get("passes") or [])
    for k in ("status", "label", "where", "case", "passes", "repeat_identical"):
        row[k] = st[k]
    counts = [c["hip_calls"] for p in log.get("passes") or [] for r in p for c in r.get("calls", [])
              if c.get("hip_calls")]
    row["allocs_per_call"] = _most(counts, "alloc")
    row["launches_per_call"] = _most(counts, "launch")
    t = (log.get("timing") or {}).get("median_ms") or {}
    k_ms = t.get("kernel")
    if row["status"] == "pass" and k_ms:
        row["kernel_ms"] = k_ms
        row["x_eager"] = round(t["eager"] / k_ms, 2) if t.get("eager") else None
        row["pct_expert"] = round(t["expert"] / k_ms * 100.0, 1) if t.get("expert") else None
    return row


def _cell(v) -> str:
    if v is None:
        return ""
    if isinstance(v, float):
        return f"{v:.4g}"
    return str(v)


def read_logs(log_dir) -> list[tuple[Path, dict]]:
    out = []
    for p in sorted(Path(log_dir).glob("*.json")):
        if p.name in OUTPUT_FILES:
            continue
        data = json.loads(p.read_text())
        if isinstance(data, dict) and "task" in data:
            out.append((p, data))
    return out


def tables(log_dir, recompute: bool = False) -> list[dict]:
    """Write verdicts.json (kernel -> row) and table.md; return the rows."""
    log_dir = Path(log_dir)
    rows = []
    for p, log in read_logs(log_dir):
        row = verdict_row(log) if recompute or "verdict" not in log else log["verdict"]
        row = dict(row, kernel=row.get("kernel") or p.stem)
        if recompute:
            log["verdict"] = row
            p.write_text(json.dumps(log, indent=1))
        rows.append(row)
    (log_dir / "verdicts.json").write_text(json.dumps({r["kernel"]: r for r in rows}, indent=1))
    lines = ["| " + " | ".join(HEADER) + " |", "|" + "|".join("---" for _ in HEADER) + "|"]
    for r in rows:
        cells = (r["kernel"], r["task"], r["status"], r["label"],
                 " / ".join(x for x in (r.get("case"), r.get("where")) if x) or None,
                 r["kernel_ms"], r["x_eager"], r["pct_expert"], r["repeat_identical"],
                 r["allocs_per_call"], r["launches_per_call"])
        lines.append("| " + " | ".join(_cell(c) for c in cells) + " |")
    (log_dir / "table.md").write_text("\n".join(lines) + "\n")
    return rows


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("action", choices=("table", "regrade"))
    ap.add_argument("log_dir")
    a = ap.parse_args(argv)
    rows = tables(a.log_dir, recompute=a.action == "regrade")
    sys.stdout.write((Path(a.log_dir) / "table.md").read_text())
    return 0 if rows else 1


if __name__ == "__main__":
    sys.exit(main())
