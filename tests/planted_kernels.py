"""Planted runners for the negative controls: each has the grader's runner interface
(`bind(arena, scalars) -> fire()`) and is wrong in one known way, so the harness must
give it one known label (graders/planted.py:10-53 names the same kinds of fault).
Not collected by pytest.

- OracleKernel (CPU): reads its inputs from a host arena, computes the outputs with the
  oracle, writes them, then plants its fault in host memory.  Used by the CPU tests.
- DeviceFault (GPU): runs the real HIP kernel through its drop-in library on a device
  arena, then plants its fault in device memory with torch's own device operations (a
  fill, a copy, an add), so the harness's device-side checks -- guard gaps, 0xFF
  outputs, unchanged inputs, call-2 results, repeat bits -- must catch it.  Every planted
  write lands inside the arena's one allocation; no GPU kernel is altered.
- PlantedLibrary (GPU): the task's planted drop-in library, lib/planted_<op>.so
  (grader/plants.py): the real entry with the fault compiled in, a HIP kernel launched
  after it (or, for a cached result, a call that returns before launching anything),
  reached through the same grader_entry ABI as the task's own library.
"""
import numpy as np
import torch

from cob_amd import tasks
from cob_amd.grader.arena import POISON_FILL
from oracle import exact

WRONG = 12345.0  # far from every op's results

# planted fault -> (status, label) the verdict must give
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


def _first_input(task):
    return next(p.name for p in task["params"] if p.pointer and p.name not in task["outputs"])


def _last_output(task):
    return [p.name for p in task["params"] if p.name in task["outputs"]][-1]


class _PerArena:
    """Calls made into each arena (one arena per graded case), and what a caching plant
    kept from the arena's first call."""

    def __init__(self):
        self.seen = {}

    def next_call(self, arena):
        entry = self.seen.setdefault(id(arena), [arena, 0, {}])   # the arena is kept alive
        entry[1] += 1
        return entry[1], entry[2]


def _plant_after(fault, arena, task, calls, cache):
    """Plant `fault` into the arena after the (correct) outputs have been written;
    `calls` counts the calls into this arena, `cache` is its own."""
    outs = arena.outputs()
    if fault == "cached_result":
        if calls == 1:
            cache.update({n: arena.view(n).clone() for n in outs})
        else:
            for n in outs:
                arena.view(n).copy_(cache[n])            # the first call's result, again
    elif fault == "wrong_value":
        arena.view(outs[0]).view(-1)[0] = WRONG
    elif fault == "oob_write_before":
        r = arena.by_name[outs[0]]
        arena.mem[r.start - 1] = 0
    elif fault == "oob_write_after":
        r = arena.by_name[_last_output(task)]
        arena.mem[r.start + r.nbytes] = 0
    elif fault == "unwritten_output":
        r = arena.by_name[_last_output(task)]
        es = arena.view(r.name).element_size()
        arena.mem[r.start + r.nbytes - es:r.start + r.nbytes] = POISON_FILL
    elif fault == "input_modified":
        r = arena.by_name[_first_input(task)]
        arena.mem[r.start] ^= 0x01
    elif fault == "nonrepeatable" and calls == 3:
        # call 3 repeats call 1's inputs; one output differs in its lowest bit
        flat = arena.view(outs[0]).view(-1)
        flat.view(torch.int16 if flat.element_size() == 2 else torch.int32)[0] ^= 1


class OracleKernel:
    """A CPU runner: the oracle's outputs, written into a host arena, then `fault`."""

    def __init__(self, op: str, fault: str | None = None):
        self.op, self.fault = op, fault
        self.task = tasks.load_task(op)
        self.arenas = _PerArena()

    def bind(self, arena, scalars):
        def fire():
            calls, cache = self.arenas.next_call(arena)
            if not (self.fault == "cached_result" and calls > 1):
                inp = dict(scalars)
                for p in self.task["params"]:
                    if p.pointer and p.name not in self.task["outputs"]:
                        t = arena.view(p.name).clone()
                        inp[p.name] = t.view(torch.float8_e4m3fn) if "fp8" in p.ctype else t
                want = exact.reference_exact(self.op, inp)
                for name in arena.outputs():
                    out = arena.view(name)
                    vals = torch.as_tensor(np.asarray(want[name], dtype=np.float64)).reshape(out.shape)
                    out.copy_(vals.to(out.dtype))
            _plant_after(self.fault, arena, self.task, calls, cache)
        return fire


class DeviceFault:
    """A GPU runner: the op's real drop-in kernel on a device arena, then `fault` planted
    in device memory by a torch device operation."""

    def __init__(self, op: str, fault: str | None = None):
        from cob_amd.grader.entry import DropInLibrary
        self.op, self.fault = op, fault
        self.task = tasks.load_task(op)
        self.lib = DropInLibrary(op)
        self.arenas = _PerArena()

    def bind(self, arena, scalars):
        kernel = self.lib.bind(arena, scalars)

        def fire():
            calls, cache = self.arenas.next_call(arena)
            if not (self.fault == "cached_result" and calls > 1):
                kernel()
            _plant_after(self.fault, arena, self.task, calls, cache)
        return fire


class PlantedLibrary:
    """A GPU runner: lib/planted_<op>.so with `fault` selected.  The library counts its
    calls from the selection (for the cached and call-3 kinds), so a runner that grades
    several cases is restarted by start_case() before each."""

    def __init__(self, op: str, fault: str | None = None):
        import ctypes
        from cob_amd import LIB_DIR
        from cob_amd.grader.entry import DropInLibrary
        from cob_amd.grader.plants import KINDS
        path = LIB_DIR / f"planted_{op}.so"
        self.lib = DropInLibrary(op, path=path)
        self._select = ctypes.CDLL(str(path)).planted_select
        self._select.argtypes = [ctypes.c_int]
        self._select.restype = None
        self._kind = KINDS.index(fault or "none")
        self._select(self._kind)

    def start_case(self):
        """Select the kind again, which restarts the library's call count: each graded case
        then sees calls 1, 2, 3 (the reference grades each case in its own process)."""
        self._select(self._kind)

    def bind(self, arena, scalars):
        return self.lib.bind(arena, scalars)
