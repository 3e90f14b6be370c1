"""One allocation per graded case holding every buffer the entry point is handed.

Layout (byte offsets; every buffer starts on a 256-byte boundary):

    | gap 0 | buffer 0 | gap 1 | buffer 1 | ... | buffer n-1 | gap n |

Each gap is at least GUARD_BYTES (4 KiB) long and filled with GUARD_FILL (0xA5), so every
buffer has 4 KiB of guard on both sides, as in the reference's harness
(graders/child.py:21-22, 52-64).  Outputs are filled with POISON_FILL (0xFF: a NaN for
fp32 and bf16) before each call; inputs hold the call's input bytes.

The arena keeps an *expected image* of itself: what every byte outside the outputs must
still hold after the call.  `strays()` compares the arena with that image in one pass and
names the region of every differing byte, so a write anywhere outside the outputs is seen
-- into a guard gap (an out-of-bounds write) or into an input (input modified) -- with
its byte offset.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

GUARD_BYTES = 4096
GUARD_FILL = 0xA5
POISON_FILL = 0xFF
ALIGN = 256


@dataclass
class Region:
    name: str
    role: str            # "in" or "out"
    start: int           # byte offset in the arena
    nbytes: int
    dtype: torch.dtype   # the element type the kernel sees
    shape: tuple


def _round_up(n: int, a: int) -> int:
    return -(-n // a) * a


def _bytes_of(t: torch.Tensor) -> torch.Tensor:
    t = t.detach().contiguous()
    if t.dtype == torch.float8_e4m3fn:
        t = t.view(torch.uint8)
    return t.reshape(-1).view(torch.uint8).cpu()


class Arena:
    """Guarded buffers for one set of arguments.  `specs` is a list of
    (name, role, dtype, shape) in the entry point's argument order."""

    def __init__(self, specs, device="cuda"):
        self.device = torch.device(device)
        self.regions: list[Region] = []
        at = GUARD_BYTES
        for name, role, dtype, shape in specs:
            n = 1
            for s in shape:
                n *= int(s)
            nbytes = n * torch.empty((), dtype=dtype).element_size()
            self.regions.append(Region(name, role, at, nbytes, dtype, tuple(int(s) for s in shape)))
            at = _round_up(at + nbytes, ALIGN) + GUARD_BYTES
        self.size = at
        self.by_name = {r.name: r for r in self.regions}
        self.mem = torch.empty(self.size, dtype=torch.uint8, device=self.device)
        self.expect = torch.empty_like(self.mem)
        # Every byte range that must not change: the gaps and the inputs, in address order.
        self.watched: list[tuple[str, int, int]] = []
        lo = 0
        for r in self.regions:
            self.watched.append((f"gap before {r.name}", lo, r.start))
            if r.role == "in":
                self.watched.append((f"input {r.name}", r.start, r.start + r.nbytes))
            lo = r.start + r.nbytes
        self.watched.append((f"gap after {self.regions[-1].name}" if self.regions else "gap", lo, self.size))

    # -- addresses and views ---------------------------------------------------------
    def address(self, name: str) -> int:
        return self.mem.data_ptr() + self.by_name[name].start

    def view(self, name: str) -> torch.Tensor:
        r = self.by_name[name]
        return self.mem[r.start:r.start + r.nbytes].view(r.dtype).view(r.shape)

    def outputs(self) -> list[str]:
        return [r.name for r in self.regions if r.role == "out"]

    # -- staging and inspection ------------------------------------------------------
    def image(self, values: dict) -> torch.Tensor:
        """The host byte image of the whole arena for one input set: guards, input bytes,
        poisoned outputs."""
        img = torch.full((self.size,), GUARD_FILL, dtype=torch.uint8)
        for r in self.regions:
            if r.role == "out":
                img[r.start:r.start + r.nbytes] = POISON_FILL
            else:
                src = _bytes_of(values[r.name])
                if src.numel() != r.nbytes:
                    raise ValueError(f"{r.name}: {src.numel()} bytes for a {r.nbytes}-byte buffer")
                img[r.start:r.start + r.nbytes] = src
        return img

    def stage(self, img: torch.Tensor) -> None:
        """Write an image into the arena and remember it as the expected state."""
        self.mem.copy_(img)
        self.expect.copy_(img)

    def strays(self) -> list[dict]:
        """Bytes outside the outputs that differ from the staged image, per watched range:
        [{"region": "gap before <name>" | "gap after <name>" | "input <name>",
          "first": byte offset in the arena, "bytes": how many differ}], in address order.
        Empty when nothing outside the outputs moved."""
        diff = self.mem != self.expect
        found = []
        for label, lo, hi in self.watched:
            if hi <= lo:
                continue
            part = diff[lo:hi]
            n = int(part.sum())
            if n:
                first = lo + int(torch.nonzero(part)[0, 0])
                found.append({"region": label, "first": first, "bytes": n})
        return found

    def snapshot(self) -> dict[str, torch.Tensor]:
        """Copies of every output as the kernel left it."""
        return {n: self.view(n).clone() for n in self.outputs()}
