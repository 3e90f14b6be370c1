"""Planted CPU kernels for the negative controls (tests/test_planted.py, tests/test_proof_flow.py):
a CPU kernel with the drop-in's bind/call interface that reads its inputs from the guarded
input buffers it is handed, computes the op with the oracle and writes the guarded output
buffers, except for one planted fault (graders/planted.py:10-53 plants the same faults in
CUDA).  Not collected by pytest."""
import numpy as np
import torch

from cob_amd import tasks
from cob_amd.grader import harness
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


