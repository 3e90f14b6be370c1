"""Planted negative controls: kernels that are wrong in one known way must draw their named
label from the same harness the real kernels are graded by (the three-call protocol on
guarded buffers, grader/harness.py check(); labels, grader/verdict.py).  Counterpart of
graders/planted.py:10-53 (EXPECT) with the labels of graders/verdict.py:35-61.

The plants run on the CPU, never as GPU code.  Each is a CPU kernel with the drop-in's
bind/call interface: it reads its inputs from the guarded input buffers it is handed,
computes the op with the oracle and writes the guarded output buffers, except for one
planted fault.  The buffers live in host memory (check(device="cpu")); everything else is
the harness the GPU tests use.

The reference's race and uninitialised-read plants have no counterpart: they are caught by
compute-sanitizer's racecheck and initcheck, and ROCm has neither.  Races are covered by
design review and the bitwise repeat check (the `nonrepeatable` plant shows that check
firing); unwritten outputs by the 0xFF poison (`unwritten_output`).
"""
import pytest

from cob_amd import tasks
from cob_amd.grader import harness
from cob_amd.grader.verdict import case_result, verdict
from oracle import exact
from planted_kernels import EXPECT, PlantedCpuKernel


def _case(op):
    return next(c for c in tasks.all_cases(op) if c["name"].startswith("public_"))


@pytest.mark.parametrize("fault", list(EXPECT))
@pytest.mark.parametrize("op", tasks.OPS)
def test_planted_control_gets_its_label(op, fault):
    case = _case(op)
    rec = harness.check(op, case, exact.reference_exact, kernel=PlantedCpuKernel(op, fault), device="cpu")
    rec["name"] = case["name"]
    v = verdict([[rec]])
    assert (v["status"], v["label"]) == EXPECT[fault], (rec.get("compare"), rec["calls"])
    if fault in (None, "wrong_value", "oob_write_before", "oob_write_after", "input_modified"):
        assert v["identical_repeat"] is True
    if fault == "nonrepeatable":
        assert v["identical_repeat"] is False


@pytest.mark.parametrize("op", ["reward_to_go", "fp8_linear"])
def test_planted_flip_between_passes(op):
    """A kernel right in one pass and wrong in the other is a flip, labelled by its failure."""
    case = _case(op)
    passes = []
    for fault in (None, "wrong_value"):
        rec = harness.check(op, case, exact.reference_exact, kernel=PlantedCpuKernel(op, fault), device="cpu")
        rec["name"] = case["name"]
        passes.append([rec])
    v = verdict(passes)
    assert (v["status"], v["label"]) == ("flip", "wrong value")
    assert v["passes"] == ["pass", "fail"]


def test_planted_failure_names_the_check():
    """The failing check names the call and buffer, as the reference's logs do."""
    op = "leaky"
    case = _case(op)
    rec = harness.check(op, case, exact.reference_exact, kernel=PlantedCpuKernel(op, "oob_write_after"), device="cpu")
    ok, chk, label = case_result(rec)
    assert (ok, chk, label) == (False, "call1:guards", "out-of-bounds write")
    rec = harness.check(op, case, exact.reference_exact, kernel=PlantedCpuKernel(op, "cached_result"), device="cpu")
    assert case_result(rec)[1].startswith("call2:")
