"""Element-wise agreement of one output with the oracle.

The rule is the tasks' own (tasks/FORMAT.md:37): an element agrees when
|got - want| <= atol + rtol * |want|, and a non-finite `want` is matched only by the same
value (NaN by NaN, +inf by +inf).  That is numpy's `isclose(got, want, rtol, atol,
equal_nan=True)` with `want` as the second argument, which is what `tally` evaluates.

Besides the count of disagreeing elements a tally reports how many of them still hold the
0xFF fill the harness writes before the call (never written by the kernel), the largest
error as a fraction of its bound, and the first disagreeing element.
"""
from __future__ import annotations

import numpy as np
import torch

UNWRITTEN = 0xFF


def _numbers(x) -> np.ndarray:
    """Any tensor or array as a flat float64 array (bf16/fp16/fp8 widened exactly)."""
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu()
        if x.dtype in (torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.bool):
            x = x.to(torch.float32)
        return x.to(torch.float64).reshape(-1).numpy()
    return np.asarray(x, dtype=np.float64).reshape(-1)


def _unwritten(got, picks: np.ndarray) -> int:
    """How many of the elements at `picks` are all-0xFF bytes."""
    if not isinstance(got, torch.Tensor) or picks.size == 0:
        return 0
    t = got.detach().cpu().contiguous()
    width = t.element_size()
    raw = t.reshape(-1).view(torch.uint8).numpy().reshape(-1, width)
    return int(np.count_nonzero(np.all(raw[picks] == UNWRITTEN, axis=1)))


def tally(got, want, tol: dict) -> dict:
    """{"elements", "size_ok", "mismatched", "unwritten", "worst", "first"} for one output.
    `worst` is max |got - want| / (atol + rtol |want|) over the elements with finite values
    (inf where a non-finite pair disagrees); `first` is {"index", "got", "want"} of the
    first disagreeing element, or None."""
    g, w = _numbers(got), _numbers(want)
    out = {"elements": int(g.size), "size_ok": g.size == w.size}
    if not out["size_ok"]:
        out.update(mismatched=int(max(g.size, w.size)), unwritten=0, worst=float("inf"), first=None)
        return out
    atol, rtol = float(tol.get("atol", 0.0)), float(tol.get("rtol", 0.0))
    agree = np.isclose(g, w, rtol=rtol, atol=atol, equal_nan=True)
    bad = np.flatnonzero(~agree)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        bound = atol + rtol * np.abs(w)
        err = np.abs(g - w)
        finite = np.isfinite(g) & np.isfinite(w)
        ratio = np.zeros_like(err)
        np.divide(err, bound, out=ratio, where=finite & (bound > 0))
        ratio[finite & (bound == 0) & (err > 0)] = np.inf
    ratio[bad[~finite[bad]]] = np.inf
    out["mismatched"] = int(bad.size)
    out["unwritten"] = _unwritten(got, bad)
    out["worst"] = float(ratio.max()) if ratio.size else 0.0
    out["first"] = None if bad.size == 0 else {"index": int(bad[0]), "got": float(g[bad[0]]),
                                                "want": float(w[bad[0]])}
    return out
