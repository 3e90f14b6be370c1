"""Source of a task's planted drop-in library: the real `reference(...)` entry of dropin.hpp
plus one known fault, chosen at run time, behind the same `grader_entry(void**)` ABI as
the task's own drop-in (graders/planted.py:10-53 names the reference's planted kinds and
their labels; there each kind is a separate CUDA build of the expert kernel).

One library per task (`lib/planted_<op>.so`) holds every kind; `planted_select(kind)`
picks one and restarts the library's call count.  The faults are HIP kernels (and one
host-side shortcut) that run after, or instead of, the real kernel on the default stream:

    kind  name               what the library does                        label
    0     none               the real kernel only                         pass
    1     wrong_value        the first output's first element := 12345    wrong value
    2     cached_result      calls after the first return at once         stale state
    3     oob_write_before   one zero byte just before the first output   out-of-bounds write
    4     oob_write_after    one zero byte just past the last output      out-of-bounds write
    5     unwritten_output   the last output's last element := 0xFF bytes unwritten output
    6     input_modified     the first input's first byte XOR 1           input modified
    7     nonrepeatable      on call 3 the first output's lowest bit flips pass, repeat bits false

The out-of-bounds kinds write one byte next to a buffer, which is only harmless where
the buffer sits inside a larger allocation, as in the harness's arena (a 4 KiB guard gap
on each side).  The library is a test control: nothing but the harness's tests loads it.
"""
from __future__ import annotations

import struct

from .signature import Param

KINDS = ("none", "wrong_value", "cached_result", "oob_write_before", "oob_write_after",
         "unwritten_output", "input_modified", "nonrepeatable")

ELEMENT_BYTES = {"float32": 4, "bfloat16": 2, "float16": 2, "float64": 8}
WRONG_VALUE = 12345.0  # far from every op's outputs


def wrong_bits(dtype: str) -> int:
    """Little-endian bits of WRONG_VALUE in `dtype` (bf16 rounded to nearest even)."""
    if dtype == "float64":
        return struct.unpack("<Q", struct.pack("<d", WRONG_VALUE))[0]
    f32 = struct.unpack("<I", struct.pack("<f", WRONG_VALUE))[0]
    if dtype == "float32":
        return f32
    if dtype == "bfloat16":
        return (f32 + 0x7FFF + ((f32 >> 16) & 1)) >> 16
    if dtype == "float16":
        return struct.unpack("<H", struct.pack("<e", WRONG_VALUE))[0]
    raise ValueError(f"no planted value for dtype {dtype}")


def _count(shape, scalars: set) -> str:
    """C++ element count of an output shape: names are scalar parameters, numbers literal."""
    terms = []
    for d in shape:
        if isinstance(d, int) or str(d).isdigit():
            terms.append(f"{int(d)}LL")
        elif d in scalars:
            terms.append(f"(long long){d}")
        else:
            raise ValueError(f"shape entry {d!r} is neither a number nor a scalar parameter")
    return " * ".join(terms) if terms else "1LL"


def planted_source(params: list[Param], outputs: dict, header: str = "dropin.hpp") -> str:
    """C++ source of the planted library for one task: `params` its signature, `outputs`
    the task's {name: {"dtype", "shape"}} in output order."""
    names = [p.name for p in params]
    out_names = [n for n in outputs if n in names]
    if not out_names:
        raise ValueError("the signature names none of the task's outputs")
    first_in = next((p for p in params if p.pointer and p.name not in outputs), None)
    if first_in is None:
        raise ValueError("the signature has no input pointer")
    scalars = {p.name for p in params if not p.pointer}
    first, last = out_names[0], out_names[-1]
    first_bytes = ELEMENT_BYTES[outputs[first]["dtype"]]
    last_bytes = ELEMENT_BYTES[outputs[last]["dtype"]]
    slots = {p.name: f"*({p.cell}*)a[{i}]" for i, p in enumerate(params)}
    lines = [
        f'#include "{header}"',
        "",
        "// Planted controls (grader/plants.py): the real entry plus the fault planted_select() picks.",
        "namespace {",
        "int g_kind = 0;   // index into grader/plants.py KINDS",
        "int g_calls = 0;  // calls since the last planted_select()",
        "",
        "__global__ void plant_bytes(unsigned char* p, unsigned long long bits, int n, int xor_mode) {",
        "  for (int i = 0; i < n; ++i) {",
        "    const unsigned char b = (unsigned char)(bits >> (8 * i));",
        "    p[i] = xor_mode ? (unsigned char)(p[i] ^ b) : b;",
        "  }",
        "}",
        "",
        "void plant(void* p, long long offset, unsigned long long bits, int n, int xor_mode) {",
        "  hipLaunchKernelGGL(plant_bytes, dim3(1), dim3(1), 0, nullptr,",
        "                     static_cast<unsigned char*>(p) + offset, bits, n, xor_mode);",
        "}",
        "}  // namespace",
        "",
        'extern "C" void planted_select(int kind) {',
        "  g_kind = kind;",
        "  g_calls = 0;",
        "}",
        "",
        'extern "C" void grader_entry(void** a) {',
        "  ++g_calls;",
        "  if (g_kind == 2 && g_calls > 1) return;  // cached_result: never recomputes",
    ]
    for p in params:
        lines.append(f"  auto&& {p.name} = {slots[p.name]};")
    lines += [
        f"  reference({', '.join(names)});",
        f"  const long long last_count = {_count(outputs[last]['shape'], scalars)};",
        "  switch (g_kind) {",
        f"    case 1: plant((void*){first}, 0, {wrong_bits(outputs[first]['dtype']):#x}ULL, {first_bytes}, 0); break;",
        f"    case 3: plant((void*){first}, -1, 0ULL, 1, 0); break;",
        f"    case 4: plant((void*){last}, last_count * {last_bytes}, 0ULL, 1, 0); break;",
        f"    case 5: if (last_count > 0) plant((void*){last}, (last_count - 1) * {last_bytes}, ~0ULL, {last_bytes}, 0); break;",
        f"    case 6: plant((void*){first_in.name}, 0, 1ULL, 1, 1); break;",
        f"    case 7: if (g_calls == 3) plant((void*){first}, 0, 1ULL, 1, 1); break;",
        "    default: break;",
        "  }",
        "}",
        "",
    ]
    return "\n".join(lines)
