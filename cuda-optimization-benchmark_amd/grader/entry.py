"""Reaching a kernel through its drop-in library's `grader_entry(void**)`.

A bound call owns one block of 8-byte cells, one per argument, and a table of the cells'
addresses.  A pointer argument's cell holds the device address; a scalar's cell holds the
value's little-endian bytes in its first 1, 4 or 8 bytes.  The shim reads slot i as
`*(T*)a[i]` (grader/signature.py), so the table is exactly what it expects.  Cells and
table stay alive as long as the bound call does.
"""
from __future__ import annotations

import ctypes
import struct

from .. import LIB_DIR
from ..tasks import load_task

# struct formats of the scalar types that appear in the task signatures
SCALAR_FORMAT = {"float": "<f", "double": "<d", "int": "<i", "int32_t": "<i", "int64_t": "<q", "bool": "<?"}


class DropInLibrary:
    """lib/dropin_<op>.so of one task.  `bind(arena, scalars)` returns a function of no
    arguments that makes the call."""

    def __init__(self, op: str, path=None):
        self.op = op
        self.params = load_task(op)["params"]
        self.path = path or (LIB_DIR / f"dropin_{op}.so")
        if not self.path.exists():
            raise RuntimeError(f"{self.path} is not built; run __graft_entry__.build() first")
        self._fn = ctypes.CDLL(str(self.path)).grader_entry
        self._fn.argtypes = [ctypes.c_void_p]
        self._fn.restype = None

    def bind(self, arena, scalars: dict):
        cells, table = pack(self.params, arena.address, scalars)
        fn = self._fn

        def fire(_keep=(cells, table)):
            fn(ctypes.addressof(table))
        return fire


def pack(params, address_of, scalars: dict):
    """(cells, table) for one call: `address_of(name)` gives a pointer argument's device
    address, `scalars[name]` a scalar's value."""
    n = max(len(params), 1)
    cells = (ctypes.c_uint64 * n)()
    for i, p in enumerate(params):
        if p.pointer:
            cells[i] = address_of(p.name)
        else:
            struct.pack_into(SCALAR_FORMAT[p.base], cells, 8 * i, scalars[p.name])
    base = ctypes.addressof(cells)
    table = (ctypes.c_void_p * n)(*[base + 8 * i for i in range(len(params))])
    return cells, table
