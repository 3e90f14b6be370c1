"""Element-wise tolerance check of one output against the oracle (graders/child.py:150-175).

Pass rule per element: |out - ref| <= atol + rtol * |ref|; where ref is not finite the
output must equal it (NaN matches NaN).  The summary counts bad elements, how many of
them still hold the 0xFF poison (an unwritten output), and the worst error as a fraction
of the bound.
"""
from __future__ import annotations

import numpy as np
import torch

POISON = 0xFF


def _as_f64(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu()
        if x.dtype in (torch.bfloat16, torch.float16, torch.float8_e4m3fn):
            x = x.float()
        return x.double().numpy().reshape(-1)
    return np.asarray(x, dtype=np.float64).reshape(-1)


def _poison_mask(out) -> np.ndarray:
    if isinstance(out, torch.Tensor):
        t = out.detach().cpu().contiguous()
        raw = t.reshape(-1).view(torch.uint8).numpy()
        n = t.numel()
    else:
        a = np.ascontiguousarray(out)
        raw = a.reshape(-1).view(np.uint8)
        n = a.size
    if n == 0:
        return np.zeros(0, dtype=bool)
    return (raw.reshape(n, -1) == POISON).all(axis=1)


def compare(out, ref, tol: dict) -> dict:
    o = _as_f64(out)
    r = _as_f64(ref)
    s = {"n": int(o.size), "shape_ok": o.size == r.size}
    if not s["shape_ok"]:
        s["bad"] = int(o.size)
        return s
    atol, rtol = float(tol.get("atol", 0.0)), float(tol.get("rtol", 0.0))
    with np.errstate(invalid="ignore", over="ignore"):
        bound = atol + rtol * np.abs(r)
        err = np.abs(o - r)
        fin = np.isfinite(r)
        ok = np.where(fin, err <= bound, (np.isnan(r) & np.isnan(o)) | (o == r))
        ratio = np.where(fin & np.isfinite(o), err / np.maximum(bound, 1e-300),
                         np.where(ok, 0.0, np.inf))
    bad = ~ok
    s["bad"] = int(bad.sum())
    s["worst"] = float(ratio.max()) if ratio.size else 0.0
    if s["bad"]:
        idx = np.nonzero(bad)[0]
        i = int(idx[0])
        s["first_bad"] = i
        s["bad_poison"] = int(_poison_mask(out)[idx].sum())
        s["example"] = {"index": i, "got": float(o[i]), "want": float(r[i])}
    return s
