"""Planted negative controls on device memory: the real HIP kernel of each op, run through
its drop-in library on a device arena, with one fault planted afterwards in device memory
(tests/planted_kernels.py DeviceFault).  The harness's device-side checks must give each
its label (graders/planted.py:16-53; results/gpu_proof.json records the reference's own
planted run):

    wrong value        one output element overwritten on the device
    cached result      call 2 rewrites call 1's device result instead of recomputing
    gap writes         one byte written into the 4 KiB guard gap before / after an output
                       (inside the arena's allocation, so nothing faults)
    unwritten output   the last output element refilled with 0xFF
    input modified     one input byte changed on the device
    nonrepeatable      call 3 differs from call 1 in one bit (a pass, repeat bits false)

test_device_plant_gets_its_label alters no GPU kernel: every plant is a torch device
operation on the arena.  test_hip_plant_gets_its_label grades the planted drop-in libraries
(lib/planted_<op>.so, grader/plants.py): the fault is a HIP kernel (or a skipped call)
behind the task's grader_entry ABI, as the reference's planted kernels are CUDA builds.
"""
import pytest

from cob_amd import tasks
from cob_amd.grader.labels import kernel_status
from cob_amd.grader.protocol import run_case
from oracle import exact
from planted_kernels import EXPECT, DeviceFault, PlantedLibrary

pytestmark = pytest.mark.gpu


def _public(op):
    return next(c for c in tasks.all_cases(op) if c["name"].startswith("public_"))


@pytest.mark.parametrize("fault", list(EXPECT))
@pytest.mark.parametrize("op", tasks.OPS)
def test_device_plant_gets_its_label(lib, op, fault):
    print(f"\n[planted] {op} {fault}", flush=True)
    report = run_case(op, _public(op), exact.reference_exact, runner=DeviceFault(op, fault))
    st = kernel_status([[report]])
    assert (st["status"], st["label"]) == EXPECT[fault], (report["checks"], report["calls"])
    assert st["repeat_identical"] is (fault != "nonrepeatable")


@pytest.mark.parametrize("fault", list(EXPECT))
@pytest.mark.parametrize("op", tasks.OPS)
def test_hip_plant_gets_its_label(lib, op, fault):
    print(f"\n[planted lib] {op} {fault}", flush=True)
    report = run_case(op, _public(op), exact.reference_exact, runner=PlantedLibrary(op, fault))
    st = kernel_status([[report]])
    assert (st["status"], st["label"]) == EXPECT[fault], (report["checks"], report["calls"])
    # a library that skips its later calls leaves call 3's outputs unwritten as well
    assert st["repeat_identical"] is (fault not in ("nonrepeatable", "cached_result"))
