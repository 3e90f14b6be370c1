"""Verdict labels from per-case records (the rules of graders/verdict.py:35-116).

Pass = every case correct on calls 1 and 2, with guards and inputs intact.  Failure
labels, in the order they are checked: timeout, cuda error, out-of-bounds write, input
modified, crash, wrong shape / unwritten output / wrong value (call 1), stale state
(call 2).  A kernel that passes some passes and fails others is a `flip`.
"""
from __future__ import annotations


def case_result(rec: dict):
    """(ok, check, label); ok is None when the process died before calling the kernel."""
    if rec.get("proc") == "timeout":
        return False, "timeout", "timeout"
    calls = rec.get("calls", [])
    for c in calls:
        if c.get("cuda_error"):
            return False, f"call{c['call']}:cuda_error", "cuda error"
        if not all(c.get("guards_ok", {}).values()):
            return False, f"call{c['call']}:guards", "out-of-bounds write"
        if not all(c.get("inputs_unchanged", {}).values()):
            return False, f"call{c['call']}:inputs", "input modified"
    if rec.get("proc") != "ok":
        return (None, "no_call", None) if not calls else (False, "crash", "crash")
    for name, s in rec["compare"]["call1"].items():
        if s["bad"]:
            if not s.get("shape_ok", True):
                return False, f"call1:{name}", "wrong shape"
            if s.get("bad_poison") == s["bad"]:
                return False, f"call1:{name}", "unwritten output"
            return False, f"call1:{name}", "wrong value"
    for name, s in rec["compare"]["call2"].items():
        if s["bad"]:
            return False, f"call2:{name}", "stale state"
    return True, None, None


def verdict(passes: list[list[dict]]) -> dict:
    """Verdict over one or more passes, each a list of case records (with `name`)."""
    v = {"status": None, "label": None, "failed_case": None, "failed_check": None,
         "identical_repeat": None, "passes": []}
    results = []
    for cases in passes:
        first = None
        for rec in cases:
            ok, chk, label = case_result(rec)
            if ok is None:
                first = ("grader_error", rec.get("name"), chk, None)
                break
            if not ok and first is None:
                first = ("timeout" if chk == "timeout" else "fail", rec.get("name"), chk, label)
        results.append(first or ("pass", None, None, None))
    v["passes"] = [r[0] for r in results]
    if not results:
        v["status"] = "grader_error"
        return v
    bad = next((r for r in results if r[0] != "pass"), None)
    if bad is None:
        v["status"] = "pass"
    elif bad[0] == "grader_error" or all(r[0] != "pass" for r in results):
        v["status"], v["failed_case"], v["failed_check"], v["label"] = bad
    else:
        v["status"], v["failed_case"], v["failed_check"], v["label"] = ("flip",) + bad[1:]
    recs = [r for cases in passes for r in cases if r.get("proc") == "ok"]
    if recs:
        v["identical_repeat"] = all(r.get("identical_repeat") for r in recs)
    return v
