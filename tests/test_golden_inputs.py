"""The package's input generators reproduce the reference's seeded inputs bit for bit.

Pinned against tests/golden/input_digests.json: SHA-256 digests of the tensors the
reference's own `make_inputs` (tasks/<id>/reference.py) returns for every hidden and
public case at both grader seeds (written by tests/golden/make_golden.py).
"""
import hashlib
import json
from pathlib import Path

import pytest
import torch

from cob_amd import inputs, tasks

GOLDEN = json.loads((Path(__file__).parent / "golden" / "input_digests.json").read_text())

# The two largest inputs (leaky T256_B512_H1024, 512 MiB; pow b16_h512_w512) are checked
# at one seed to keep the CPU suite short; every other case at both seeds.
_CASES = []
for op in tasks.OPS:
    for key in sorted(GOLDEN[op]):
        name, seed = key.rsplit("@", 1)
        big = name in ("T256_B512_H1024", "b16_h512_w512", "B4096_I256_O512", "M2048_K1024_N4096")
        case = next(c for c in tasks.all_cases(op) if c["name"] == name)
        if big and int(seed) != int(case["seed"]):
            continue
        _CASES.append((op, key))


def _digest(v):
    if isinstance(v, torch.Tensor):
        t = v.contiguous()
        raw = t.reshape(-1).view(torch.uint8).numpy().tobytes()
        return {"dtype": str(t.dtype), "shape": list(t.shape), "sha256": hashlib.sha256(raw).hexdigest()}
    return {"scalar": v}


@pytest.mark.parametrize("op,key", _CASES)
def test_inputs_match_reference(op, key):
    name, seed = key.rsplit("@", 1)
    case = next(c for c in tasks.all_cases(op) if c["name"] == name)
    got = inputs.make_inputs(op, case, int(seed))
    want = GOLDEN[op][key]
    assert set(got) == set(want)
    for k, v in got.items():
        assert _digest(v) == want[k], (op, key, k)


def test_every_case_has_a_digest():
    for op in tasks.OPS:
        names = {k.rsplit("@", 1)[0] for k in GOLDEN[op]}
        assert names == {c["name"] for c in tasks.all_cases(op)}
