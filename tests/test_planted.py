"""Planted negative controls on the CPU: a runner that is wrong in one known way must draw
its named label from the same protocol, arena and label rules the HIP kernels are graded
by (grader/protocol.py, grader/labels.py).  The counterpart of graders/planted.py:10-53.

Here the runners are tests/planted_kernels.py's OracleKernel: the oracle's outputs
written into a host arena, with one fault planted afterwards.  tests/test_planted_device.py
plants the same faults in device memory around the real HIP kernels.

The reference's race and uninitialised-read plants have no counterpart: they are caught by
compute-sanitizer's racecheck and initcheck, which ROCm lacks.  Races are covered by design
review and the bitwise repeat check (the `nonrepeatable` plant shows it firing), and
unwritten outputs by the 0xFF fill (`unwritten_output`).
"""
import pytest

from cob_amd import tasks
from cob_amd.grader.labels import case_outcome, kernel_status
from cob_amd.grader.protocol import run_case
from oracle import exact
from planted_kernels import EXPECT, OracleKernel


def _public(op):
    return next(c for c in tasks.all_cases(op) if c["name"].startswith("public_"))


def _grade(op, fault):
    return run_case(op, _public(op), exact.reference_exact, runner=OracleKernel(op, fault), device="cpu")


@pytest.mark.parametrize("fault", list(EXPECT))
@pytest.mark.parametrize("op", tasks.OPS)
def test_planted_control_gets_its_label(op, fault):
    report = _grade(op, fault)
    st = kernel_status([[report]])
    assert (st["status"], st["label"]) == EXPECT[fault], (report["checks"], report["calls"])
    assert st["repeat_identical"] is (fault != "nonrepeatable")


@pytest.mark.parametrize("op", ["reward_to_go", "fp8_linear"])
def test_right_then_wrong_is_a_flip(op):
    passes = [[_grade(op, None)], [_grade(op, "wrong_value")]]
    st = kernel_status(passes)
    assert (st["status"], st["label"], st["passes"]) == ("flip", "wrong value", ["pass", "fail"])


def test_failure_names_the_call_and_region():
    """The location names the call, the region and the first byte that moved."""
    op = "leaky"
    o = case_outcome(_grade(op, "oob_write_after"))
    assert o["label"] == "out-of-bounds write" and o["where"].startswith("call 1: gap after final_mem (byte ")
    o = case_outcome(_grade(op, "oob_write_before"))
    assert o["where"].startswith("call 1: gap before spikes")
    o = case_outcome(_grade(op, "input_modified"))
    assert o["where"].startswith("call 1: input input_current")
    o = case_outcome(_grade(op, "cached_result"))
    assert (o["label"], o["where"]) == ("stale state", "call 2: spikes")
    o = case_outcome(_grade(op, "unwritten_output"))
    assert (o["label"], o["where"]) == ("unwritten output", "call 1: final_mem")
