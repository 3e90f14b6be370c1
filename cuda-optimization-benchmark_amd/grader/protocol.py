"""The graded run of one case: three calls into one arena.

The calls (the reference's protocol, graders/child.py:178-215, stated as a schedule):

    call 1  input set A (the case's seed)          judged against the oracle
    call 2  input set B (seed + 7919), same buffers  judged against the oracle
    call 3  input set A again                       must reproduce call 1's bits

Before every call the whole arena is rewritten from its image for that input set (guards,
inputs, 0xFF outputs), so a kernel that keeps results from an earlier call is caught on
call 2 (its outputs still fit set A) and one that leaves outputs unwritten shows 0xFF.
After every call the device is synchronised (an asynchronous fault surfaces here), the
arena is checked for bytes that moved outside the outputs, and the outputs are copied.

The report of a case (JSON-ready):

    {"case": name, "state": "finished" | "crashed" | "not started" | "timeout",
     "calls":  [{"call": 1, "inputs": "A", "host_ms": t, "strays": [...], "error": str,
                 "hip_calls": {category: count}}, ...],
     "checks": {"1": {output: tally}, "2": {output: tally}},   # grader/tolerance.py
     "repeat_identical": bool}

`checker(op, inputs) -> {output: array}` computes the expected outputs (the caller passes
the oracle); `runner` is anything with `bind(arena, scalars) -> fire()`, by default the
task's drop-in library (grader/entry.py).
"""
from __future__ import annotations

import time
from dataclasses import dataclass

import torch

from ..capi import output_shapes
from ..inputs import make_inputs
from ..tasks import SET_B, load_task
from .arena import Arena
from .tolerance import tally


@dataclass(frozen=True)
class Call:
    number: int
    inputs: str      # "A" or "B"
    judged: bool


SCHEDULE = (Call(1, "A", True), Call(2, "B", True), Call(3, "A", False))
REPEAT_OF = {3: 1}   # call -> the earlier call whose output bits it must reproduce


def input_sets(op: str, case: dict) -> dict:
    seed = int(case["seed"])
    return {"A": make_inputs(op, case, seed), "B": make_inputs(op, case, seed + SET_B)}


def arena_specs(op: str, inp: dict) -> list[tuple]:
    """(name, role, dtype, shape) for every pointer argument, in signature order."""
    task = load_task(op)
    shapes = output_shapes(op, inp)
    specs = []
    for p in task["params"]:
        if not p.pointer:
            continue
        if p.name in task["outputs"]:
            shape, dtype = shapes[p.name]
            specs.append((p.name, "out", dtype, shape))
        else:
            t = inp[p.name]
            dtype = torch.uint8 if t.dtype == torch.float8_e4m3fn else t.dtype
            specs.append((p.name, "in", dtype, list(t.shape)))
    return specs


def scalar_args(op: str, inp: dict) -> dict:
    return {p.name: inp[p.name] for p in load_task(op)["params"] if not p.pointer}


def _settle(device: torch.device):
    """Wait for the device; the text of an asynchronous error, or None."""
    if device.type != "cuda":
        return None
    try:
        torch.cuda.synchronize()
    except RuntimeError as e:
        return str(e)[:400]
    return None


def run_case(op: str, case: dict, checker, runner=None, device="cuda", hip_calls=None, sets=None) -> dict:
    """Grade one case; see the module text for the report.  `hip_calls(fire) -> dict`, when
    given, makes the call and returns the HIP runtime calls it made (callcount.py)."""
    if runner is None:
        from .entry import DropInLibrary
        runner = DropInLibrary(op)
    tol = load_task(op)["tolerance"]
    sets = sets or input_sets(op, case)
    arena = Arena(arena_specs(op, sets["A"]), device)
    images = {k: arena.image(v) for k, v in sets.items()}
    report = {"case": case["name"], "state": "not started", "calls": [], "checks": {},
              "repeat_identical": None}
    kept = {}
    for call in SCHEDULE:
        arena.stage(images[call.inputs])
        fire = runner.bind(arena, scalar_args(op, sets[call.inputs]))
        if _settle(arena.device) is not None:      # staging itself failed: nothing was graded
            return report
        obs = {"call": call.number, "inputs": call.inputs}
        report["state"] = "crashed"                # until the call is seen to complete
        t0 = time.perf_counter()
        counts = hip_calls(fire) if hip_calls else fire()
        obs["host_ms"] = round((time.perf_counter() - t0) * 1e3, 4)
        if hip_calls:
            obs["hip_calls"] = counts
        report["calls"].append(obs)
        err = _settle(arena.device)
        if err is not None:
            obs["error"] = err
            return report
        obs["strays"] = arena.strays()
        kept[call.number] = arena.snapshot()
    report["repeat_identical"] = all(
        torch.equal(kept[a][n].reshape(-1).view(torch.uint8), kept[b][n].reshape(-1).view(torch.uint8))
        for a, b in REPEAT_OF.items() for n in kept[a])
    for call in SCHEDULE:
        if call.judged:
            want = checker(op, sets[call.inputs])
            report["checks"][str(call.number)] = {n: tally(got, want[n], tol) for n, got in kept[call.number].items()}
    report["state"] = "finished"
    return report


def time_case(op: str, case: dict, eager=None, runner=None, rounds: int = 3) -> dict:
    """The kernel's ms per call on set A in a staged arena and, when `eager(op, inputs)` is
    given, the PyTorch eager reference's on the same inputs on the GPU, alternated over
    `rounds` rounds (grader/clock.py race)."""
    from .clock import race
    if runner is None:
        from .entry import DropInLibrary
        runner = DropInLibrary(op)
    inp = make_inputs(op, case, int(case["seed"]))
    arena = Arena(arena_specs(op, inp), "cuda")
    arena.stage(arena.image(inp))
    sides = {"kernel": runner.bind(arena, scalar_args(op, inp))}
    if eager is not None:
        dev = {k: (v.to("cuda") if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
        sides["eager"] = lambda: eager(op, dev)
    res = race(sides, rounds=rounds)
    res.update(case=case["name"], gpu=torch.cuda.get_device_name(), torch=torch.__version__)
    return res
