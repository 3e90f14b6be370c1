"""Write tests/golden/input_digests.json from the reference's own input generators.

Run in the build container only (it needs /root/reference, which the GPU box does not
have):  python tests/golden/make_golden.py

The reference's `make_inputs(case, seed, device)` (tasks/<id>/reference.py) is the one
function of the path that no closed form or invariant can pin: bitwise identity of the
seeded inputs depends on the RNG draw order, the fp32 rounding of scalars and the
float8 cast.  For every hidden and public case and both seeds the grader uses (seed,
seed + 7919), this records the SHA-256 of each tensor's bytes with its dtype and shape,
and every scalar.  tests/test_golden_inputs.py checks the package's restated
generators against these digests.  Nothing else of the reference is run.
"""
from __future__ import annotations

import hashlib
import importlib.util
import json
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
REF = Path("/root/reference/tasks")
SET_B = 7919
OPS = ["pow_abs_sqrt_mean", "leaky", "reward_to_go", "ppo_clip", "efficient_kan", "fp8_linear"]


def _module(op: str):
    spec = importlib.util.spec_from_file_location(f"ref_{op}", REF / op / "reference.py")
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def digest(v):
    if isinstance(v, torch.Tensor):
        t = v.contiguous()
        raw = t.reshape(-1).view(torch.uint8).numpy().tobytes()
        return {"dtype": str(t.dtype), "shape": list(t.shape), "sha256": hashlib.sha256(raw).hexdigest()}
    return {"scalar": v}


def main() -> int:
    out = {}
    for op in OPS:
        m = _module(op)
        cases = json.loads((REF / op / "tests" / "task.json").read_text())["cases"]
        public = json.loads((REF / op / "environment" / "public_cases.json").read_text())["cases"]
        rec = {}
        for prefix, group in (("", cases), ("public_", public)):
            for case in group:
                for off in (0, SET_B):
                    seed = int(case["seed"]) + off
                    inp = m.make_inputs(case, seed, "cpu")
                    rec[f"{prefix}{case['name']}@{seed}"] = {k: digest(v) for k, v in inp.items()}
        out[op] = rec
        print(op, len(rec), flush=True)
    (HERE / "input_digests.json").write_text(json.dumps(out, indent=1, sort_keys=True))
    return 0


if __name__ == "__main__":
    sys.exit(main())
