"""The C ABI from plain C: tests/c_abi_call.c includes include/taskops.h and the HIP runtime
API only, and is compiled by gcc as C11 with warnings as errors, linked against
lib/libtaskops.so and libamdhip64.  On the CPU the build is the test (the header is valid C
and every symbol the program uses links); on the GPU the program runs reward_to_go through the
C ABI on a created stream and checks every output, in a child process of its own."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

from cob_amd import LIB_DIR

ROOT = Path(__file__).resolve().parents[1]
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def _build(out: Path) -> Path:
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    if not (LIB_DIR / "libtaskops.so").exists():
        pytest.fail("lib/libtaskops.so is not built")
    exe = out / "c_abi_call"
    cmd = ["gcc", "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROOT / 'include'}", f"-I{ROCM / 'include'}", str(ROOT / "tests" / "c_abi_call.c"),
           "-o", str(exe), f"-L{LIB_DIR}", "-ltaskops", f"-L{ROCM / 'lib'}", "-lamdhip64", "-lm",
           f"-Wl,-rpath,{LIB_DIR}", f"-Wl,-rpath,{ROCM / 'lib'}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def test_c_caller_builds(tmp_path):
    _build(tmp_path)


@pytest.mark.gpu
def test_c_caller_runs(tmp_path):
    exe = _build(tmp_path)
    print("\n[capi] plain C caller: reward_to_go B=37 T=1031", flush=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout, r.stderr)
