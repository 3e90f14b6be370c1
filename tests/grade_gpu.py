"""Grade the six drop-in kernels and every planted library on one GPU, and write one log
per kernel, the tables and the proof record (the role of graders/grade.py + child.py,
and of grade.py's `proof`, graders/grade.py:228-253; logs and tables by
grader/ledger.py).  Not collected by pytest; run as

    python tests/grade_gpu.py OUT_DIR [--ops a,b] [--passes 2] [--no-timing] [--no-planted]

For each op (grade_op()): every hidden and public case through the three-call protocol on
a device arena (grader/protocol.py run_case), in `--passes` passes, with the HIP call
counter armed around each call; then the task's timed case, kernel against PyTorch eager
on the same GPU in alternating rounds (protocol.time_case).  Then each op's planted
library, lib/planted_<op>.so, once per planted kind (grader/plants.py KINDS): every
case in one pass, no timing, as the reference grades its planted kernels.  proof.json
holds every drop-in's verdict, every plant's expected and actual verdict, and the counts
{references_pass, planted_as_expected}; proof.md is the same as a table.
tests/test_proof_flow.py runs grade_op() and proof() on the CPU with planted runners.
The checker is oracle/exact.py and the eager side oracle/eager.py, which is why this
driver lives under tests/.  No expert (reference CUDA) kernel runs on this GPU, so
"% of expert" stays empty.
"""
import argparse
import json
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
import __graft_entry__  # noqa: E402

__graft_entry__.load_package()
from cob_amd import callcount  # noqa: E402


def grade_op(op, runner, checker, passes=2, hip_calls=None, device="cuda", eager=None, key=None, env=None,
             log=print):
    """One kernel's log: every hidden and public case of `op` in `passes` passes, then
    (with `eager`) the timed case's timing, and the verdict row."""
    from cob_amd import tasks
    from cob_amd.grader import ledger
    from cob_amd.grader.protocol import run_case, time_case
    t0 = time.time()
    entry = {"kernel": key or f"taskops_{op}", "task": op, "env": env or {}, "build": {"ok": True},
             "passes": []}
    for p in range(passes):
        reports = []
        for case in tasks.all_cases(op):
            log(f"[grade] {op} pass {p + 1} {case['name']}")
            if hasattr(runner, "start_case"):
                runner.start_case()  # a planted library restarts its call count per case
            reports.append(run_case(op, case, checker, runner=runner, device=device, hip_calls=hip_calls))
        entry["passes"].append(reports)
    if eager is not None:
        timed = next(c for c in tasks.all_cases(op) if c.get("timed"))
        log(f"[grade] {op} timing {timed['name']}")
        entry["timing"] = time_case(op, timed, eager=eager, runner=runner)
    entry["wall_s"] = round(time.time() - t0, 2)
    entry["verdict"] = ledger.verdict_row(entry)
    return entry


def _expected_ok(kind, row, expect) -> bool:
    """Whether a planted library's verdict row is the one its kind must draw: the expected
    (status, label), and for the kinds that pass, the expected repeat bits (false only
    for the plant whose call 3 differs)."""
    status, label = expect
    if (row.get("status"), row.get("label")) != (status, label):
        return False
    return status != "pass" or row.get("repeat_identical") is (kind != "nonrepeatable")


def proof(rows: dict, references: dict, planted: dict, expect: dict, env: dict) -> dict:
    """The proof record (graders/grade.py:228-253): `rows` maps kernel keys to verdict
    rows; `references` maps each op to its drop-in's key; `planted` maps "op/kind" to
    (key, kind); `expect` maps a kind (None for "none") to its (status, label)."""
    res = {"gpu": env.get("gpu"), "env": env, "references": {}, "planted": {}}
    for op, key in references.items():
        r = rows.get(key, {})
        res["references"][op] = {k: r.get(k) for k in ("status", "label", "case", "kernel_ms", "x_eager",
                                                        "repeat_identical", "allocs_per_call", "launches_per_call")}
    for name, (key, kind) in planted.items():
        r = rows.get(key, {})
        want = expect[None if kind == "none" else kind]
        res["planted"][name] = {"expect": f"{want[0]} / {want[1]}", "status": r.get("status"),
                                "label": r.get("label"), "repeat_identical": r.get("repeat_identical"),
                                "ok": _expected_ok(kind, r, want)}
    res["summary"] = {
        "references_pass": sum(v["status"] == "pass" and v["repeat_identical"] is True
                               for v in res["references"].values()),
        "references": len(res["references"]),
        "planted_as_expected": sum(v["ok"] for v in res["planted"].values()),
        "planted": len(res["planted"])}
    return res


def proof_table(res: dict) -> str:
    """proof.json as markdown: the drop-ins, then every plant with its expected verdict."""
    s = res["summary"]
    lines = [f"references_pass {s['references_pass']}/{s['references']}, "
             f"planted_as_expected {s['planted_as_expected']}/{s['planted']}", "",
             "| drop-in | status | label | identical repeat | kernel ms | x eager |", "|---|---|---|---|---:|---:|"]
    num = lambda x: "" if x is None else f"{x:.4g}"
    for op, v in res["references"].items():
        lines.append(f"| {op} | {v['status']} | {v['label'] or ''} | {v['repeat_identical']} | "
                     f"{num(v['kernel_ms'])} | {num(v['x_eager'])} |")
    lines += ["", "| planted library / kind | expected | status | label | identical repeat | as expected |",
              "|---|---|---|---|---|---|"]
    for name, v in res["planted"].items():
        lines.append(f"| {name} | {v['expect']} | {v['status']} | {v['label'] or ''} | {v['repeat_identical']} | "
                     f"{'yes' if v['ok'] else 'NO'} |")
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("out_dir")
    ap.add_argument("--ops", default="")
    ap.add_argument("--passes", type=int, default=2)
    ap.add_argument("--no-timing", action="store_true")
    ap.add_argument("--no-planted", action="store_true", help="grade the drop-ins only")
    a = ap.parse_args(argv)
    counter = callcount.load_counter()  # before torch loads the HIP runtime

    import torch
    from cob_amd import LIB_DIR, tasks
    from cob_amd.grader import ledger
    from cob_amd.grader.entry import DropInLibrary
    from oracle import eager, exact
    if not torch.cuda.is_available():
        print("grade_gpu.py needs a GPU", file=sys.stderr)
        return 1
    torch.backends.cuda.matmul.allow_tf32 = False  # the graded process's setting (child.py:29-30)
    out = Path(a.out_dir)
    out.mkdir(parents=True, exist_ok=True)
    ops = [o for o in a.ops.split(",") if o] or tasks.OPS
    env = {"gpu": torch.cuda.get_device_name(), "arch": getattr(torch.cuda.get_device_properties(0), "gcnArchName", ""),
           "torch": torch.__version__, "python": platform.python_version()}
    (out / "env.json").write_text(json.dumps(env, indent=1))
    for op in ops:
        lib = LIB_DIR / f"dropin_{op}.so"
        if lib.exists():
            entry = grade_op(op, DropInLibrary(op), exact.reference_exact, passes=a.passes,
                             hip_calls=lambda fire: counter.count(fire, 0),
                             eager=None if a.no_timing else eager.reference, env=env,
                             log=lambda m: print(m, file=sys.stderr, flush=True))
            entry["build"] = {"ok": True, "lib": lib.name, "tail": ""}
        else:
            entry = {"kernel": f"taskops_{op}", "task": op, "env": env, "passes": [],
                     "build": {"ok": False, "lib": lib.name, "tail": f"{lib} not built"}}
            entry["verdict"] = ledger.verdict_row(entry)
        (out / f"{entry['kernel']}.json").write_text(json.dumps(entry, indent=1))
        v = entry["verdict"]
        print(f"[grade] {op}: {v['status']} {v['label'] or ''} kernel {v['kernel_ms']} ms, "
              f"x{v['x_eager']} vs eager", file=sys.stderr, flush=True)
    planted = {}
    if not a.no_planted:
        from cob_amd.grader.plants import KINDS
        from planted_kernels import PlantedLibrary
        for op in ops:
            for kind in KINDS:
                key = f"planted_{op}__{kind}"
                entry = grade_op(op, PlantedLibrary(op, kind), exact.reference_exact, passes=1,
                                 hip_calls=lambda fire: counter.count(fire, 0), eager=None, key=key, env=env,
                                 log=lambda m: None)
                entry["build"] = {"ok": True, "lib": f"planted_{op}.so", "tail": ""}
                (out / f"{key}.json").write_text(json.dumps(entry, indent=1))
                planted[f"{op}/{kind}"] = (key, kind)
                v = entry["verdict"]
                print(f"[grade] planted {op}/{kind}: {v['status']} {v['label'] or ''}", file=sys.stderr, flush=True)
    rows = {r["kernel"]: r for r in ledger.tables(out)}
    print((out / "table.md").read_text(), end="")
    if planted:
        from planted_kernels import EXPECT
        res = proof(rows, {op: f"taskops_{op}" for op in ops}, planted, EXPECT, env)
        (out / "proof.json").write_text(json.dumps(res, indent=1))
        (out / "proof.md").write_text(proof_table(res))
        print(json.dumps(res["summary"]), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
