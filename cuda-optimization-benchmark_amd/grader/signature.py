"""A task's C++ entry signature as data, and the text of its `grader_entry` shim.

The signature strings are the tasks' own (tasks/<id>/tests/task.json:3).  The shim is the
calling convention the reference's ctypes driver expects of a drop-in library
(graders/grade.py:85-89): one `extern "C" void grader_entry(void** a)` whose slot `a[i]`
holds the address of argument i -- for a pointer argument the address of a cell holding
the pointer, for a scalar the address of a cell holding the value.
"""
from __future__ import annotations

import re
from dataclasses import dataclass

# Words and stars of a C declaration; nothing else appears in the task signatures.
_TOKEN = re.compile(r"\*|[A-Za-z_][A-Za-z0-9_]*")


@dataclass(frozen=True)
class Param:
    """One parameter: its name and its C type as written (qualifiers kept, spacing
    normalised so that `const float *x` and `const float* x` give "const float*")."""
    name: str
    ctype: str

    @property
    def pointer(self) -> bool:
        return self.ctype.endswith("*")

    @property
    def base(self) -> str:
        """The value type without qualifiers or indirection ("float", "__hip_bfloat16")."""
        words = [w for w in self.ctype.replace("*", " ").split() if w not in ("const", "volatile")]
        return " ".join(words)

    @property
    def cell(self) -> str:
        """The type the shim reads slot i as: the declared type for pointers; for scalars
        the declared type with its top-level `const` removed (a cell is writable)."""
        if self.pointer:
            return self.ctype
        return " ".join(w for w in self.ctype.split() if w != "const")


def parse(signature: str) -> list[Param]:
    """The parameters of `void reference(...)`, in order.  Raises ValueError when the text
    has no `reference(...)` or a parameter has no name."""
    at = signature.find("reference")
    if at < 0 or "(" not in signature[at:]:
        raise ValueError(f"not a reference(...) signature: {signature!r}")
    open_ = signature.index("(", at)
    close = signature.rindex(")")
    params = []
    for chunk in signature[open_ + 1:close].split(","):
        tokens = _TOKEN.findall(chunk)
        if not tokens:
            continue
        if tokens[-1] == "*":
            raise ValueError(f"unnamed parameter {chunk.strip()!r}")
        *words, name = tokens
        stars = words.count("*")
        params.append(Param(name, " ".join(w for w in words if w != "*") + "*" * stars))
    return params


def shim(params: list[Param], header: str = "dropin.hpp") -> str:
    """C++ source of the drop-in entry: `header` stands where the reference's shim
    includes the kernel's source file."""
    slots = [f"*({p.cell}*)a[{i}]" for i, p in enumerate(params)]
    return (f'#include "{header}"\n'
            f'extern "C" void grader_entry(void** a) {{ reference({", ".join(slots)}); }}\n')
