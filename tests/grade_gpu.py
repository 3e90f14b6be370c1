"""Grade the six drop-in kernels on one GPU and write one log per kernel plus the tables
(the role of graders/grade.py + child.py; logs and tables by grader/ledger.py).  Not
collected by pytest; run as

    python tests/grade_gpu.py OUT_DIR [--ops a,b] [--passes 2] [--no-timing]

For each op (grade_op()): every hidden and public case through the three-call protocol on
a device arena (grader/protocol.py run_case), in `--passes` passes, with the HIP call
counter armed around each call; then the task's timed case, kernel against PyTorch eager
on the same GPU in alternating rounds (protocol.time_case).  tests/test_proof_flow.py
runs grade_op() on the CPU with planted runners.  The checker is oracle/exact.py and the
eager side oracle/eager.py, which is why this driver lives under tests/.  No expert
(reference CUDA) kernel runs on this GPU, so "% of expert" stays empty.
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
            reports.append(run_case(op, case, checker, runner=runner, device=device, hip_calls=hip_calls))
        entry["passes"].append(reports)
    if eager is not None:
        timed = next(c for c in tasks.all_cases(op) if c.get("timed"))
        log(f"[grade] {op} timing {timed['name']}")
        entry["timing"] = time_case(op, timed, eager=eager, runner=runner)
    entry["wall_s"] = round(time.time() - t0, 2)
    entry["verdict"] = ledger.verdict_row(entry)
    return entry


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("out_dir")
    ap.add_argument("--ops", default="")
    ap.add_argument("--passes", type=int, default=2)
    ap.add_argument("--no-timing", action="store_true")
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
    ledger.tables(out)
    print((out / "table.md").read_text(), end="")
    return 0


if __name__ == "__main__":
    sys.exit(main())
