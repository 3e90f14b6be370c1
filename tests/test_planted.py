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
import numpy as np
import pytest
import torch

from cob_amd import tasks
from cob_amd.grader import harness
from cob_amd.grader.verdict import case_result, verdict
from oracle import exact

WRONG = 12345.0  # far from every op's results

# plant -> (status, label) the verdict must give
EXPECT = {
    None: ("pass", None),
    "wrong_value": ("fail", "wrong value"),
    "cached_result": ("fail", "stale state"),
    "oob_write_before": ("fail", "out-of-bounds write"),
    "oob_write_after": ("fail", "out-of-bounds write"),
    "unwritten_output": ("fail", "unwritten output"),
    "input_modified": ("fail", "input modified"),
    "nonrepeatable": ("pass", None),
}


class PlantedCpuKernel:
    """A CPU kernel behind DropIn's interface; `fault` names the planted mistake."""

    def __init__(self, op: str, fault: str | None = None):
        self.op, self.fault = op, fault
        self.task = tasks.load_task(op)
        self.calls = 0

    def bind(self, bufs: dict, scalars: dict):
        return (bufs, scalars), None

    def _inputs(self, bufs, scalars) -> dict:
        inp = dict(scalars)
        for ctype, name in self.task["params"]:
            if "*" in ctype and name not in self.task["outputs"]:
                t = bufs[name].t.clone()
                inp[name] = t.view(torch.float8_e4m3fn) if "fp8" in ctype else t
        return inp

    def __call__(self, arr) -> None:
        bufs, scalars = arr
        self.calls += 1
        if self.fault == "cached_result" and self.calls > 1:
            return  # assumes the inputs never change between calls
        want = exact.reference_exact(self.op, self._inputs(bufs, scalars))
        for name in self.task["outputs"]:
            out = bufs[name].t
            flat = out.view(-1)
            flat.copy_(torch.as_tensor(np.asarray(want[name], dtype=np.float64)).reshape(-1).to(out.dtype))
            g = harness.GUARD
            if self.fault == "wrong_value":
                flat[0] = WRONG
            elif self.fault == "oob_write_before":
                bufs[name].raw[g - 1] = 0
            elif self.fault == "oob_write_after":
                bufs[name].raw[g + bufs[name].n] = 0
            elif self.fault == "unwritten_output":
                es = flat.element_size()
                bufs[name].raw[g + bufs[name].n - es:g + bufs[name].n] = harness.POISON
            elif self.fault == "nonrepeatable" and self.calls == 3:
                # call 3 repeats call 1's inputs; one output differs by one unit in the last place
                flat.view(torch.int16 if flat.element_size() == 2 else torch.int32)[0] ^= 1
        if self.fault == "input_modified":
            name = next(n for c, n in self.task["params"] if "*" in c and n not in self.task["outputs"])
            bufs[name].raw[harness.GUARD] ^= 0x01


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
