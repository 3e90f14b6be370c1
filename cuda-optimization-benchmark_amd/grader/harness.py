"""The graded process on device memory: guarded buffers, the three-call protocol, and
hipEvent timing (the HIP counterpart of graders/child.py).

- Guarded: every input and output lives inside a device allocation with 4 KiB of 0xA5
  guard bytes on each side (child.py:52-64); outputs are filled with 0xFF (NaN for fp32
  and bf16) before each call.
- check(): call 1 with the case's seed, call 2 with seed + 7919 written into the same
  buffers, call 3 with the first values again (child.py:178-215); after each call the
  guards and the inputs are checked, and calls 1 and 2 are compared with the injected
  `exact` checker under the task tolerance.  Identical bits on call 3 are reported.
- events(): median ms per call from hipEvents around back-to-back calls (child.py:228-244);
  timing() runs it in interleaved rounds for the kernel and the PyTorch eager reference
  (child.py:247-265).

The kernel is reached the way the reference's grader reaches it: `grader_entry(void**)`
of the op's drop-in library (lib/dropin_<op>.so), with argument addresses bound from the
task signature (child.py:79-100).
"""
from __future__ import annotations

import ctypes
import statistics
import time

import torch

from .. import LIB_DIR
from ..capi import output_shapes, DTYPES
from ..inputs import make_inputs
from ..tasks import SET_B, load_task
from .compare import compare

GUARD = 4096
GUARD_BYTE = 0xA5
POISON = 0xFF

CTYPES = {"float": ctypes.c_float, "double": ctypes.c_double, "int": ctypes.c_int,
          "int32_t": ctypes.c_int32, "int64_t": ctypes.c_int64, "bool": ctypes.c_bool}


def _raw(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().reshape(-1).view(torch.uint8)


class Guarded:
    """A device buffer fenced by guard bytes; `.t` is the tensor the kernel sees."""

    def __init__(self, nbytes: int, dtype: torch.dtype, shape, device="cuda"):
        self.n = nbytes
        self.raw = torch.full((GUARD + nbytes + GUARD,), GUARD_BYTE, dtype=torch.uint8, device=device)
        self.t = self.raw[GUARD:GUARD + nbytes].view(dtype).view(shape)

    def guards_ok(self) -> bool:
        return bool((self.raw[:GUARD] == GUARD_BYTE).all() and (self.raw[GUARD + self.n:] == GUARD_BYTE).all())

    def poison(self) -> None:
        self.raw[GUARD:GUARD + self.n].fill_(POISON)

    def load(self, src: torch.Tensor) -> None:
        self.raw[GUARD:GUARD + self.n].copy_(_raw(src))

    def same_as(self, src: torch.Tensor) -> bool:
        return bool(torch.equal(self.raw[GUARD:GUARD + self.n], _raw(src).to(self.raw.device)))


class DropIn:
    """One op's drop-in library, called through its `grader_entry(void**)` shim."""

    def __init__(self, op: str, path=None):
        self.task = load_task(op)
        p = path or (LIB_DIR / f"dropin_{op}.so")
        if not p.exists():
            raise RuntimeError(f"{p} is not built; run __graft_entry__.build() first")
        self.fn = ctypes.CDLL(str(p)).grader_entry
        self.fn.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.fn.restype = None

    def bind(self, bufs: dict, scalars: dict):
        keep, addrs = [], []
        for ctype, name in self.task["params"]:
            if "*" in ctype:
                v = ctypes.c_void_p(bufs[name].t.data_ptr())
            else:
                base = " ".join(w for w in ctype.split() if w != "const")
                v = CTYPES[base](scalars[name])
            keep.append(v)
            addrs.append(ctypes.addressof(v))
        return (ctypes.c_void_p * len(addrs))(*addrs), keep

    def __call__(self, arr) -> None:
        self.fn(arr)


def _buffers(task, op, inp, device="cuda"):
    bufs, outs = {}, []
    shapes = output_shapes(op, inp)
    for ctype, name in task["params"]:
        if "*" not in ctype:
            continue
        if name in task["outputs"]:
            shape, dt = shapes[name]
            n = 1
            for s in shape:
                n *= s
            bufs[name] = Guarded(n * torch.empty((), dtype=dt).element_size(), dt, shape, device)
            outs.append(name)
        else:
            x = inp[name]
            dt = torch.uint8 if x.dtype == torch.float8_e4m3fn else x.dtype
            bufs[name] = Guarded(x.numel() * x.element_size(), dt, list(x.shape), device)
    return bufs, outs


def _load_set(bufs, outs, inp):
    for name, b in bufs.items():
        if name in outs:
            b.poison()
        else:
            b.load(inp[name])
    return {k: v for k, v in inp.items() if not isinstance(v, torch.Tensor)}


def _sync(device: str) -> None:
    if device != "cpu":
        torch.cuda.synchronize()


def check(op: str, case: dict, exact, kernel: DropIn | None = None, device: str = "cuda",
          counter=None) -> dict:
    """The three-call protocol for one case; `exact(op, inputs) -> {name: array}` is the
    checker.  Returns a record shaped like the reference's per-case log.  `kernel` is
    anything with DropIn's bind/call interface; device="cpu" puts the guarded buffers in
    host memory (for CPU kernels, such as the planted controls).  `counter(fn) -> dict`,
    when given, counts the HIP calls of each kernel call into the record's `count`
    (child.py:172-178; see callcount.py)."""
    task = load_task(op)
    k = kernel or DropIn(op)
    sets = [make_inputs(op, case, int(case["seed"]) + s) for s in (0, SET_B)]
    bufs, outs = _buffers(task, op, sets[0], device)
    res = {"mode": "check", "case": case["name"], "calls": []}
    got = {}
    for call, which in ((1, 0), (2, 1), (3, 0)):
        scalars = _load_set(bufs, outs, sets[which])
        _sync(device)
        arr, keep = k.bind(bufs, scalars)
        t0 = time.time()
        count = counter(lambda: k(arr)) if counter else k(arr)
        rec = {"call": call, "host_ms": round((time.time() - t0) * 1e3, 4)}
        if counter:
            rec["count"] = count
        try:
            _sync(device)
        except RuntimeError as e:  # the context is gone: record and stop
            rec["cuda_error"] = str(e)[:300]
            res["calls"].append(rec)
            res["proc"] = "crash"
            return res
        rec["guards_ok"] = {n: b.guards_ok() for n, b in bufs.items()}
        rec["inputs_unchanged"] = {n: b.same_as(sets[which][n]) for n, b in bufs.items() if n not in outs}
        got[call] = {n: bufs[n].t.clone() for n in outs}
        res["calls"].append(rec)
    res["identical_repeat"] = all(torch.equal(_raw(got[1][n]), _raw(got[3][n])) for n in outs)
    res["compare"] = {}
    for call, which in ((1, 0), (2, 1)):
        want = exact(op, sets[which])
        res["compare"][f"call{call}"] = {n: compare(got[call][n], want[n], task["tolerance"]) for n in outs}
    res["proc"] = "ok"
    res["finished"] = True
    return res


def timing(op: str, case: dict, torch_ref=None, kernel: DropIn | None = None, rounds: int = 3) -> dict:
    """Median ms per call of the kernel and, when `torch_ref(op, inputs)` is given, of the
    PyTorch eager reference on the same device inputs: `rounds` rounds, each timing every
    side with events() in turn, then the median over rounds and the spread (max/min - 1)
    (child.py:247-265).  The kernel runs on guarded buffers, as in check()."""
    task = load_task(op)
    k = kernel or DropIn(op)
    inp = make_inputs(op, case, int(case["seed"]))
    bufs, outs = _buffers(task, op, inp)
    scalars = _load_set(bufs, outs, inp)
    arr, keep = k.bind(bufs, scalars)
    sides = {"kernel": lambda: k(arr)}
    if torch_ref is not None:
        dev = {n: (v.to("cuda") if isinstance(v, torch.Tensor) else v) for n, v in inp.items()}
        sides["torch"] = lambda: torch_ref(op, dev)
    per_round = [{n: events(f)[0] for n, f in sides.items()} for _ in range(rounds)]
    med = {n: statistics.median(r[n] for r in per_round) for n in sides}
    spread = {n: (max(r[n] for r in per_round) / min(r[n] for r in per_round) - 1)
              if min(r[n] for r in per_round) > 0 else None for n in sides}
    return {"mode": "time", "case": case["name"], "rounds": per_round, "median_ms": med, "spread": spread,
            "gpu": torch.cuda.get_device_name(), "torch": torch.__version__, "finished": True}


def events(fn, min_ms: float = 1.0, batches: int = 10, warmup: int = 3):
    """Median ms per call: hipEvents around K back-to-back calls, K chosen so one batch
    takes at least min_ms (K <= 1000).  Events are recorded on torch's current stream,
    which is the stream `fn` must launch on."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    fn()
    e1.record()
    e1.synchronize()
    one = e0.elapsed_time(e1)
    kk = max(1, min(1000, int(min_ms / one) + 1)) if one > 0 else 1000
    per = []
    for _ in range(batches):
        e0.record()
        for _ in range(kk):
            fn()
        e1.record()
        e1.synchronize()
        per.append(e0.elapsed_time(e1) / kk)
    return statistics.median(per), kk
