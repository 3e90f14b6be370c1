"""Grade the six drop-in kernels the way the reference's grader does, on one GPU, and write
one log per kernel plus the tables (graders/grade.py + child.py; tables by
cuda-optimization-benchmark_amd/grader/report.py).  Not collected by pytest; run as

    python tests/grade_gpu.py OUT_DIR [--ops a,b] [--passes 2]

For each op (grade_op()): every hidden and public case through the three-call protocol on
guarded buffers (grader/harness.py check()), in `--passes` passes, with the HIP call counter
armed around each call; then the task's timed case in 3 interleaved rounds of the kernel
and PyTorch eager on the GPU (harness.timing()).  tests/test_proof_flow.py runs grade_op()
on the CPU with planted kernels.  The checker is oracle/exact.py and the eager
side oracle/eager.py, which is why this driver lives under tests/.  There is no expert
kernel on this GPU, so `% of expert speed` stays empty.
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


def grade_op(op, kernel, exact_fn, passes=2, counter=None, device="cuda", torch_ref=None, key=None, env=None,
             log=print):
    """One kernel's grading log: every hidden and public case of `op` through check() in
    `passes` passes, then (with `torch_ref`) the timed case's timing, and the verdict."""
    from cob_amd import tasks
    from cob_amd.grader import harness, report
    t0 = time.time()
    out = {"key": key or f"taskops_{op}", "task": op, "env": env or {}, "compile": {"ok": True}, "passes": []}
    for p in range(passes):
        cases = []
        for case in tasks.all_cases(op):
            log(f"[grade] {op} pass {p + 1} {case['name']}")
            rec = harness.check(op, case, exact_fn, kernel=kernel, device=device, counter=counter)
            rec["name"] = case["name"]
            cases.append(rec)
        out["passes"].append({"cases": cases})
    if torch_ref is not None:
        timed = next(c for c in tasks.all_cases(op) if c.get("timed"))
        log(f"[grade] {op} timing {timed['name']}")
        out["timing"] = harness.timing(op, timed, torch_ref=torch_ref, kernel=kernel)
    out["seconds"] = round(time.time() - t0, 2)
    out["verdict"] = report.kernel_verdict(out)
    return out


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
    from cob_amd.grader import harness, report
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
            log = grade_op(op, harness.DropIn(op), exact.reference_exact, passes=a.passes,
                           counter=lambda fn: counter.count(fn, 0),
                           torch_ref=None if a.no_timing else eager.reference, env=env,
                           log=lambda m: print(m, file=sys.stderr, flush=True))
            log["compile"] = {"ok": True, "lib": lib.name, "log_tail": ""}
        else:
            log = {"key": f"taskops_{op}", "task": op, "env": env,
                   "compile": {"ok": False, "lib": lib.name, "log_tail": f"{lib} not built"}}
            log["verdict"] = report.kernel_verdict(log)
        (out / f"{log['key']}.json").write_text(json.dumps(log, indent=1))
        v = log["verdict"]
        print(f"[grade] {op}: {v['status']} {v['label'] or ''} kernel {v['kernel_ms']} ms, "
              f"x{v['speedup_vs_torch']} vs torch", file=sys.stderr, flush=True)
    report.write_tables(out)
    print((out / "table.md").read_text(), end="")
    return 0


if __name__ == "__main__":
    sys.exit(main())
