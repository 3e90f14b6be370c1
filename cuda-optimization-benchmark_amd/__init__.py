"""MI355X (gfx950) task-op library: the six ops of the cuda-optimization-benchmark as
hand-written HIP kernels behind a C ABI (include/taskops.h).

Modules: tasks (task specs and cases), inputs (seeded input generators), capi (ctypes
binding of libtaskops.so), grader (guarded buffers, three-call protocol, compare,
timing, verdicts), build (hipcc build of lib/*.so)."""
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_DIR = PKG_DIR / "lib"

from . import tasks  # noqa: E402,F401
