"""Milliseconds per call from hipEvents, the way the reference's grader times a kernel
(graders/child.py:228-265): back-to-back calls on unchanged buffers, batches long enough
to hide event resolution, the median over batches, and rounds that alternate between the
sides being compared so that clock drift hits every side alike.

A batch's length is found by doubling: 1, 2, 4, ... calls until one batch lasts at least
`floor_ms` (at most `cap` calls).  Events are recorded on torch's current stream, which is
the stream the timed function must launch on (the drop-in libraries use the default
stream, which is torch's current stream unless a caller changed it).
"""
from __future__ import annotations

import statistics

import torch


def _batch_ms(fn, reps: int) -> float:
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop)


def ms_per_call(fn, floor_ms: float = 1.0, samples: int = 10, warm: int = 3, cap: int = 1024) -> dict:
    """{"ms": median per-call time, "reps": calls per batch, "samples": per-call times}."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    reps = 1
    while reps < cap and _batch_ms(fn, reps) < floor_ms:
        reps *= 2
    reps = min(reps, cap)
    per = [_batch_ms(fn, reps) / reps for _ in range(samples)]
    return {"ms": statistics.median(per), "reps": reps, "samples": per}


def race(sides: dict, rounds: int = 3, **kw) -> dict:
    """Time every side once per round, sides alternating within a round.  Returns the
    per-round times, the median over rounds per side and each side's relative range
    ((max - min) / median over the rounds)."""
    table = []
    for _ in range(rounds):
        table.append({name: ms_per_call(fn, **kw)["ms"] for name, fn in sides.items()})
    median = {n: statistics.median(r[n] for r in table) for n in sides}
    spread = {}
    for n in sides:
        vals = [r[n] for r in table]
        spread[n] = (max(vals) - min(vals)) / median[n] if median[n] > 0 else None
    return {"rounds": table, "median_ms": median, "range": spread}
