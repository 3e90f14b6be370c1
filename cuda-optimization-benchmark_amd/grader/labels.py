"""Failure labels of a graded case, and the status of a kernel over several passes.

The label vocabulary is the reference's (graders/verdict.py:35-61), because its users read
these words: timeout, cuda error, out-of-bounds write, input modified, crash, wrong shape,
unwritten output, wrong value, stale state; a kernel that passes some passes and fails
others is a flip.  Here each label is one rule over the case report of
grader/protocol.py, and the rules are tried in the order of RULES: the first that finds
something names the failure and where it was seen.
"""
from __future__ import annotations


def _per_call(test):
    """A rule that applies `test(call record) -> str | None` to each call in turn."""
    def rule(report):
        for c in report.get("calls", []):
            found = test(c)
            if found:
                return f"call {c['call']}: {found}"
        return None
    return rule


def _stray_in(prefix):
    def test(c):
        hit = next((s for s in c.get("strays") or [] if s["region"].startswith(prefix)), None)
        return None if hit is None else f"{hit['region']} (byte {hit['first']}, {hit['bytes']} bytes)"
    return test


def _judged(call, test):
    """A rule over the tallies of one judged call."""
    def rule(report):
        for name, t in (report.get("checks") or {}).get(str(call), {}).items():
            if test(t):
                return f"call {call}: {name}"
        return None
    return rule


def _state(*states):
    return lambda report: report.get("state") if report.get("state") in states else None


RULES = (
    ("timeout", _state("timeout")),
    ("cuda error", _per_call(lambda c: c.get("error"))),
    ("out-of-bounds write", _per_call(_stray_in("gap"))),
    ("input modified", _per_call(_stray_in("input"))),
    ("crash", _state("crashed")),
    ("wrong shape", _judged(1, lambda t: not t["size_ok"])),
    ("unwritten output", _judged(1, lambda t: t["mismatched"] > 0 and t["unwritten"] == t["mismatched"])),
    ("wrong value", _judged(1, lambda t: t["mismatched"] > 0)),
    ("stale state", _judged(2, lambda t: t["mismatched"] > 0)),
)


def case_outcome(report: dict) -> dict:
    """{"outcome": "pass" | "fail" | "timeout" | "grader_error", "label", "where"} of one
    case.  A case that never reached its first call is a grader error (nothing of the
    kernel was seen)."""
    if report.get("state") == "not started" or (report.get("state") != "timeout" and not report.get("calls")):
        return {"outcome": "grader_error", "label": None, "where": "before call 1"}
    for label, rule in RULES:
        where = rule(report)
        if where:
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
