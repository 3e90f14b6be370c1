"""Signature parsing and the `grader_entry` shim text.

Behaviour follows graders/grade.py:73-89: a task's C++ signature is split into
(c type, name) pairs, and the shim unpacks an array of argument addresses into a call of
`reference(...)` — pointers are passed as the address of the pointer, scalars as the
address of the value with one leading `const` dropped.
"""
from __future__ import annotations

import re

_IDENT = re.compile(r"[A-Za-z_]\w*")


def parse_signature(sig: str) -> list[tuple[str, str]]:
    """[(c type, name)] of `void reference(...)`, in parameter order."""
    m = re.search(r"\breference\s*\((.*)\)", sig, re.S)
    if m is None:
        raise ValueError(f"no reference(...) in {sig!r}")
    params = []
    for part in m.group(1).split(","):
        part = " ".join(part.split())
        if not part:
            continue
        name = _IDENT.findall(part)[-1]
        params.append((part[: part.rindex(name)].strip(), name))
    return params


def _arg(ctype: str, i: int) -> str:
    if "*" in ctype:
        return f"*({ctype}*)a[{i}]"
    return f"*({ctype.replace('const ', '', 1)}*)a[{i}]"


def shim_source(params: list[tuple[str, str]], include: str = "dropin.hpp") -> str:
    """Source of the extern "C" entry for one task; `include` stands where the
    reference's shim includes `solution.cu`."""
    args = ", ".join(_arg(c, i) for i, (c, _) in enumerate(params))
    return (f'#include "{include}"\n'
            f'extern "C" void grader_entry(void** a) {{ reference({args}); }}\n')
