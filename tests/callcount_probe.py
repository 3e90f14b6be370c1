"""Subprocess helper of tests/test_callcount.py (not collected by pytest): loads the HIP
call counter before any HIP runtime, then the runtime, and calls hooks directly.  On a host
without a GPU every forwarded call returns the runtime's own error code, which shows the
call reached the runtime.  Prints one JSON object.

    python tests/callcount_probe.py counts | late_load
"""
import ctypes
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
import __graft_entry__  # noqa: E402

__graft_entry__.load_package()
from cob_amd import callcount  # noqa: E402

RUNTIME = "/opt/rocm/lib/libamdhip64.so.7"


def counts() -> dict:
    c = callcount.load_counter()
    ctypes.CDLL(RUNTIME, mode=ctypes.RTLD_GLOBAL)
    h = c.lib
    h.hipMemsetAsync.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p]
    h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    h.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
    h.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    rc = {}
    out = {"categories": c.categories}

    def on_s():  # everything on the null stream, which is the caller's stream here
        p = ctypes.c_void_p()
        rc["malloc"] = h.hipMalloc(ctypes.byref(p), ctypes.c_size_t(64))
        rc["free"] = h.hipFree(None)
        rc["memset_async"] = h.hipMemsetAsync(None, 0, 0, None)
        rc["h2d"] = h.hipMemcpy(None, None, 0, 1)
        rc["d2h_async"] = h.hipMemcpyAsync(None, None, 0, 2, None)
        rc["d2d_async"] = h.hipMemcpyAsync(None, None, 0, 3, None)
        rc["device_sync"] = h.hipDeviceSynchronize()
        rc["null_stream_sync"] = h.hipStreamSynchronize(None)

    out["on_s"] = c.count(on_s, 0)

    def off_s():  # the caller's stream is another one: null-stream work is "other stream"
        h.hipMemsetAsync(None, 0, 0, None)
        h.hipMemcpyAsync(None, None, 0, 3, None)
        h.hipMemcpy(None, None, 0, 3)

    out["off_s"] = c.count(off_s, 0x40)
    h.hipcount_reset()
    h.hipMemsetAsync(None, 0, 0, None)  # not armed: not counted
    buf = (ctypes.c_long * len(c.categories))()
    h.hipcount_read(buf, len(c.categories))
    out["disarmed"] = list(buf)
    out["rc"] = rc
    return out


def late_load() -> dict:
    ctypes.CDLL(RUNTIME, mode=ctypes.RTLD_GLOBAL)
    try:
        callcount.load_counter()
    except callcount.CallCountError as e:
        return {"refused": True, "message": str(e)}
    return {"refused": False}


if __name__ == "__main__":
    print(json.dumps({"counts": counts, "late_load": late_load}[sys.argv[1]]()))
