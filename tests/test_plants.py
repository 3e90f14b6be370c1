"""The planted drop-in sources (grader/plants.py) on the CPU: the planted bits are the
value they claim in each output dtype, the element counts follow the task's output
shapes, and every kind the tests expect a label for exists.  The GPU grading of the built
libraries is tests/test_planted_device.py."""
import re

import pytest
import torch

from cob_amd import tasks
from cob_amd.grader import plants
from cob_amd.grader.signature import parse
from planted_kernels import EXPECT


@pytest.mark.parametrize("dtype,tdt", [("float32", torch.float32), ("bfloat16", torch.bfloat16),
                                       ("float16", torch.float16), ("float64", torch.float64)])
def test_wrong_bits_are_the_value_in_that_dtype(dtype, tdt):
    want = torch.tensor(plants.WRONG_VALUE, dtype=torch.float64).to(tdt)
    raw = want.reshape(1).view(torch.uint8).tolist()
    assert plants.wrong_bits(dtype) == sum(b << (8 * i) for i, b in enumerate(raw))
    assert abs(float(want) - plants.WRONG_VALUE) < 64   # still far from every op's outputs


def test_every_expected_kind_is_built():
    assert [k or "none" for k in EXPECT] == list(plants.KINDS)


def _source(op):
    task = tasks.load_task(op)
    return plants.planted_source(parse(task["hip_signature"]), task["outputs"]), task


@pytest.mark.parametrize("op", tasks.OPS)
def test_source_targets_the_task_outputs(op):
    src, task = _source(op)
    outs = list(task["outputs"])
    first, last = outs[0], outs[-1]
    count = re.search(r"last_count = (.*);", src).group(1)
    shape = task["outputs"][last]["shape"]
    if not shape:
        assert count == "1LL"
    for d in shape:
        assert (f"(long long){d}" if isinstance(d, str) else f"{d}LL") in count
    assert f"case 1: plant((void*){first}, 0," in src
    assert f"case 4: plant((void*){last}, last_count *" in src
    assert "if (g_kind == 2 && g_calls > 1) return;" in src
    # the real entry is called with every parameter, in signature order
    names = [p.name for p in parse(task["hip_signature"])]
    assert f"reference({', '.join(names)});" in src


def test_shape_names_must_be_scalars():
    params = parse("void reference(const float* x, int n, float* out);")
    with pytest.raises(ValueError):
        plants.planted_source(params, {"out": {"dtype": "float32", "shape": ["m"]}})
