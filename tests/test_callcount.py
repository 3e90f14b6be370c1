"""HIP API call counter (csrc/callcount.c -> lib/libhipcount.so; the reference's
graders/interpose.c:14-115 armed around the graded call, graders/child.py:103-118) and the
per-call contract of every entry point it measures on the GPU.

CPU tests check the counter itself in fresh processes: hooks count by category, forward to
the runtime, honour arming, and refuse to load after the runtime.  The GPU test runs
cuda-optimization-benchmark_amd/callcount.py over every hidden and public case and checks
each steady call: no allocation, host copy, synchronisation, memset, device copy or work
off the caller's stream, and the expected number of kernel launches.
"""
import ctypes
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "cuda-optimization-benchmark_amd" / "lib" / "libhipcount.so"
PROBE = Path(__file__).resolve().parent / "callcount_probe.py"
CATEGORIES = ["alloc", "host_copy", "device_sync", "other_stream", "stream_sync", "launch", "memset", "device_copy"]
HOOKS = ["hipMalloc", "hipFree", "hipHostMalloc", "hipMallocAsync", "hipFreeAsync", "hipMemcpy", "hipMemcpyAsync",
         "hipMemcpyHtoD", "hipMemcpyDtoH", "hipMemcpyDtoD", "hipMemcpy2DAsync", "hipMemcpyToSymbolAsync",
         "hipMemset", "hipMemsetAsync", "hipMemsetD32Async", "hipDeviceSynchronize", "hipStreamSynchronize",
         "hipLaunchKernel", "hipExtLaunchKernel", "hipModuleLaunchKernel", "hipLaunchCooperativeKernel",
         "hipLaunchKernelExC", "hipGraphLaunch"]


def _probe(mode: str) -> dict:
    r = subprocess.run([sys.executable, str(PROBE), mode], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_counter_library_exports():
    lib = ctypes.CDLL(str(LIB))  # local scope: interposes nothing in this process
    for name in ["hipcount_arm", "hipcount_reset", "hipcount_read", "hipcount_set_stream", "hipcount_names"] + HOOKS:
        assert hasattr(lib, name), name
    lib.hipcount_names.restype = ctypes.c_char_p
    assert lib.hipcount_names().decode().split(",") == CATEGORIES


def test_counter_counts_classifies_and_forwards():
    out = _probe("counts")
    on_s = out["on_s"]
    assert on_s == {"alloc": 2, "host_copy": 2, "device_sync": 2, "other_stream": 0, "stream_sync": 0,
                    "launch": 0, "memset": 1, "device_copy": 1}
    # Null-stream work counted as off the caller's stream: the async memset and copy, and
    # the synchronous device copy.
    assert out["off_s"]["other_stream"] == 3 and out["off_s"]["memset"] == 1 and out["off_s"]["device_copy"] == 2
    assert out["disarmed"] == [0] * len(CATEGORIES)
    # Every call reached the runtime: without a GPU each returns the same non-zero code.
    codes = set(out["rc"].values())
    assert len(codes) == 1 and 0 not in codes and 302 not in codes, out["rc"]


def test_counter_refuses_to_load_after_the_runtime():
    out = _probe("late_load")
    assert out["refused"], out


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_entry_points_per_call_contract(tmp_path):
    """Every entry point, every case: steady calls allocate nothing, copy nothing to or from
    the host, never synchronise, put all work on the caller's stream, and launch a fixed
    number of kernels; a first call allocates at most the op's workspace."""
    print("\n[callcount] all workloads", flush=True)
    js = tmp_path / "calls.json"
    r = subprocess.run([sys.executable, "-u", str(ROOT / "cuda-optimization-benchmark_amd" / "callcount.py"),
                        "--json", str(js), "--calls", "3"], capture_output=True, text=True, timeout=540)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
    res = json.loads(js.read_text())["workloads"]
    assert len(res) >= 50
    bad = []
    for name, w in res.items():
        pc, first = w["per_call"], w["first"]
        want = dict.fromkeys(CATEGORIES, 0.0)
        want["launch"] = float(w["expect_launches"])
        if pc != want:
            bad.append((name, "steady", pc))
        if first["alloc"] > 1 or first["other_stream"] or first["host_copy"] or first["device_sync"] \
                or first["stream_sync"] or first["memset"] or first["device_copy"] \
                or first["launch"] not in (w["expect_launches"], w["expect_launches"] + 1):
            bad.append((name, "first", first))
    assert not bad, bad
