"""Build libtaskops.so (all kernels + the C ABI of include/taskops.h), the per-op
drop-in libraries for gfx950 with hipcc, the HIP call counter (libhipcount.so, gcc) and
the torch.ops.taskops operators (libtaskops_torch.so, g++), in-tree under `lib/`.

    __graft_entry__.build()   (the package directory name is not an importable identifier;
                               __graft_entry__.load_package() imports it as `cob_amd`)

The drop-in libraries (`lib/dropin_<op>.so`) each hold the C++ `void reference(...)`
overload of one task plus the grader's `extern "C" void grader_entry(void**)` shim,
linked against libtaskops.so, so the reference benchmark's ctypes driver
(graders/child.py:79-100) can load one per task unchanged.  `lib/planted_<op>.so` is the
same entry with planted faults (grader/plants.py), the harness's negative controls.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
OBJ = PKG / "_build"
INCLUDE = ROOT / "include"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-fp32 VALU forms are disabled for all device code (they have given silently
# wrong results on this pool); hipcc's host pass warns that it does not know the feature.
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}", f"-I{CSRC}",
]

# Per-file extra flags.  leaky must not contract beta*mem + x into an FMA: the spec
# rounds every operation (the source also sets `#pragma clang fp contract(off)`).
EXTRA = {
    "leaky.hip": ["-ffp-contract=off"],
}

KERNEL_SOURCES = [
    "runtime.hip",
    "pow_abs_sqrt_mean.hip",
    "ppo_clip.hip",
    "reward_to_go.hip",
    "leaky.hip",
    "efficient_kan.hip",
    "fp8_linear.hip",
    "quantize_e4m3.hip",
]

OPS = ["pow_abs_sqrt_mean", "leaky", "reward_to_go", "ppo_clip", "efficient_kan", "fp8_linear"]

# The HIP call counter is host code only: gcc, HIP headers, no HIP runtime link.
CC = os.environ.get("CC", "gcc")
COUNTER_CFLAGS = ["-O2", "-std=gnu11", "-shared", "-fPIC", "-Wall", "-Wno-deprecated-declarations",
                  "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    r = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def _compile(src: str) -> Path:
    out = OBJ / (Path(src).stem + ".o")
    cmd = [HIPCC, *COMMON, *EXTRA.get(src, []), "-c", str(CSRC / src), "-o", str(out)]
    _run(cmd)
    return out


def dropin_source(op: str) -> str:
    """The grader shim for one op (the calling convention of graders/grade.py:85-89),
    generated from the task's HIP signature, with dropin.hpp standing in for solution.cu."""
    from .grader.signature import parse, shim
    from .tasks import load_task
    return shim(parse(load_task(op)["hip_signature"]))


def planted_source(op: str) -> str:
    """The planted-control variant of an op's drop-in (grader/plants.py)."""
    from .grader.plants import planted_source as source
    from .grader.signature import parse
    from .tasks import load_task
    task = load_task(op)
    return source(parse(task["hip_signature"]), task["outputs"])


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 and link lib/libtaskops.so plus the drop-ins."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJ.mkdir(parents=True, exist_ok=True)
    LIB.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, KERNEL_SOURCES))
    lib = LIB / "libtaskops.so"
    tmp = LIB / "libtaskops.so.tmp"
    _run([HIPCC, *COMMON, "-shared", "-o", str(tmp), *map(str, objs), "-Wl,-Bsymbolic"])
    os.replace(tmp, lib)

    def _entry(name: str, text: str) -> Path:
        src = OBJ / f"{name}.hip"
        src.write_text(text)
        out = LIB / f"{name}.so"
        t = LIB / f"{name}.so.tmp"
        _run([HIPCC, *COMMON, "-shared", "-o", str(t), str(src), f"-L{LIB}", "-ltaskops",
              "-Wl,-rpath,$ORIGIN", "-Wl,-Bsymbolic"])
        os.replace(t, out)
        return out

    entries = [(f"dropin_{op}", dropin_source(op)) for op in OPS] + \
              [(f"planted_{op}", planted_source(op)) for op in OPS]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda e: _entry(*e), entries))
    counter = LIB / "libhipcount.so"
    _run([CC, *COUNTER_CFLAGS, str(CSRC / "callcount.c"), "-o", str(LIB / "libhipcount.so.tmp"), "-ldl"])
    os.replace(LIB / "libhipcount.so.tmp", counter)
    ext = build_torch_ops()
    if verbose:
        print(f"built {lib}, {len(OPS)} drop-in and {len(OPS)} planted libraries, {counter.name} and {ext.name}",
              flush=True)
    return lib


def build_torch_ops() -> Path:
    """lib/libtaskops_torch.so: the torch.ops.taskops operators (host C++ over the C ABI,
    g++ against torch's headers; libtaskops.so is found next to it)."""
    import torch
    import torch.utils.cpp_extension as ce
    out = LIB / "libtaskops_torch.so"
    tmp = LIB / "libtaskops_torch.so.tmp"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = [f"-I{p}" for p in ce.include_paths(device_type="cuda")]
    libdirs = [f"-L{p}" for p in ce.library_paths(device_type="cuda")]
    _run([os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__",
          f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_API_INCLUDE_EXTENSION_H", *inc, f"-I{INCLUDE}",
          str(CSRC / "torch_ext" / "taskops_torch.cpp"), "-o", str(tmp), *libdirs, "-lc10", "-lc10_hip",
          "-ltorch_cpu", "-ltorch_hip", "-lamdhip64", f"-L{LIB}", "-ltaskops", "-Wl,-rpath,$ORIGIN", "-Wl,--no-undefined"])
    os.replace(tmp, out)
    return out


