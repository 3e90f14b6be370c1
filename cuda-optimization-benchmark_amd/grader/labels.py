"""Failure labels of a graded case, and the status of a kernel over several passes.

The label vocabulary is the reference's (graders/verdict.py:35-61), because its users read
these words: timeout, cuda error, out-of-bounds write, input modified, crash, wrong shape,
unwritten output, wrong value, stale state; a kernel that passes some passes and fails
others is a flip.  The report is read in stages (STAGES), as the reference reads its case
record: the process state, then each call in call order with that call's own checks in the
order cuda error, out-of-bounds write, input modified, then the process state again, then
each output of judged call 1 (wrong shape, unwritten output, wrong value) and each output
of judged call 2 (stale state).  The first check that finds something names the failure
and where it was seen, so an input changed on call 1 outranks a guard hit on call 2.
"""
from __future__ import annotations


def _state(label, *states):
    """A stage that fires when the report's process state is one of `states`."""
    def stage(report):
        return (label, report.get("state")) if report.get("state") in states else None
    return stage


def _each_call(*checks):
    """A stage that walks the calls in order and tries each call's `(label, test(call
    record) -> str | None)` checks in turn."""
    def stage(report):
        for c in report.get("calls", []):
            for label, test in checks:
                found = test(c)
                if found:
                    return label, f"call {c['call']}: {found}"
        return None
    return stage


def _stray_in(prefix):
    def test(c):
        hit = next((s for s in c.get("strays") or [] if s["region"].startswith(prefix)), None)
        return None if hit is None else f"{hit['region']} (byte {hit['first']}, {hit['bytes']} bytes)"
    return test


def _each_output(call, *checks):
    """A stage over the tallies of one judged call: for each output that disagrees, in
    output order, the first `(label, test(tally))` that holds names it."""
    def stage(report):
        for name, t in (report.get("checks") or {}).get(str(call), {}).items():
            if t["mismatched"] > 0 or not t["size_ok"]:
                label = next((lab for lab, test in checks if test(t)), checks[-1][0])
                return label, f"call {call}: {name}"
        return None
    return stage


STAGES = (
    _state("timeout", "timeout"),
    _each_call(("cuda error", lambda c: c.get("error")),
               ("out-of-bounds write", _stray_in("gap")),
               ("input modified", _stray_in("input"))),
    _state("crash", "crashed"),
    _each_output(1, ("wrong shape", lambda t: not t["size_ok"]),
                 ("unwritten output", lambda t: t["unwritten"] == t["mismatched"]),
                 ("wrong value", lambda t: True)),
    _each_output(2, ("stale state", lambda t: True)),
)

# Every label a stage can give, in the order a single call's (or output's) checks try them.
LABELS = ("timeout", "cuda error", "out-of-bounds write", "input modified", "crash", "wrong shape",
          "unwritten output", "wrong value", "stale state")


def case_outcome(report: dict) -> dict:
    """{"outcome": "pass" | "fail" | "timeout" | "grader_error", "label", "where"} of one
    case.  A case that never reached its first call is a grader error (nothing of the
    kernel was seen)."""
    if report.get("state") == "not started" or (report.get("state") != "timeout" and not report.get("calls")):
        return {"outcome": "grader_error", "label": None, "where": "before call 1"}
    for stage in STAGES:
        found = stage(report)
        if found:
            label, where = found
            return {"outcome": "timeout" if label == "timeout" else "fail", "label": label, "where": where}
    return {"outcome": "pass", "label": None, "where": None}


def pass_outcome(reports: list[dict]) -> dict:
    """The first case that did not pass, in case order, or a pass."""
    for r in reports:
        o = case_outcome(r)
        if o["outcome"] != "pass":
            return dict(o, case=r.get("case"))
    return {"outcome": "pass", "label": None, "where": None, "case": None}


def kernel_status(passes: list[list[dict]]) -> dict:
    """Status over passes of the same cases: "pass" when every pass passes; the first
    failure's own outcome when every pass fails or a pass could not grade; otherwise
    "flip" with the first failure's label.  Also whether every finished case repeated its
    bits on call 3."""
    per_pass = [pass_outcome(p) for p in passes]
    status = {"status": "grader_error", "label": None, "where": None, "case": None,
              "passes": [o["outcome"] for o in per_pass], "repeat_identical": None}
    finished = [r for p in passes for r in p if r.get("state") == "finished"]
    if finished:
        status["repeat_identical"] = all(r.get("repeat_identical") for r in finished)
    if not per_pass:
        return status
    failed = [o for o in per_pass if o["outcome"] != "pass"]
    if not failed:
        status["status"] = "pass"
        return status
    lead = failed[0]
    mixed = len(failed) < len(per_pass) and lead["outcome"] != "grader_error"
    status.update(status="flip" if mixed else lead["outcome"], label=lead["label"], where=lead["where"],
                  case=lead["case"])
    return status
