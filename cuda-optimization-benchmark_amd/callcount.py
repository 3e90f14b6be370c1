"""HIP API calls made by each libtaskops entry point, per call, measured on the GPU.

    python cuda-optimization-benchmark_amd/callcount.py [--json OUT] [--calls K] [--only SUBSTR]

The counter is lib/libhipcount.so (csrc/callcount.c), the counterpart of the reference's
call interposer (graders/interpose.c:14-115, armed around the graded call as in
graders/child.py:103-118).  It must be loaded with RTLD_GLOBAL before the process loads the
HIP runtime, so this runs as its own process: load the counter, then import torch, then
call every workload through the C ABI on a created (non-default) stream with the counter
armed.

For every workload it reports the first call in the process (which may allocate the op's
cached workspace and zero it with one extra launch) and the average over K further calls,
in the categories `CATEGORIES`.  The contract the tests check on the steady calls: no
allocation, host copy, synchronisation, memset, device copy or work off the given stream,
and a fixed number of kernel launches per entry point.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
from pathlib import Path

if __package__ in (None, ""):
    # Run as a script: import the package under its importable name without torch.
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    import __graft_entry__
    __graft_entry__.load_package()
    from cob_amd import LIB_DIR
else:
    from . import LIB_DIR

LIBNAME = "libhipcount.so"


class CallCountError(RuntimeError):
    pass


def hip_runtime_loaded() -> bool:
    with open(f"/proc/{os.getpid()}/maps") as f:
        return any("libamdhip64" in line for line in f)


class Counter:
    """ctypes handle on libhipcount.so's control functions."""

    def __init__(self, lib: ctypes.CDLL):
        self.lib = lib
        lib.hipcount_arm.argtypes = [ctypes.c_int]
        lib.hipcount_set_stream.argtypes = [ctypes.c_void_p]
        lib.hipcount_read.argtypes = [ctypes.POINTER(ctypes.c_long), ctypes.c_int]
        lib.hipcount_read.restype = ctypes.c_int
        lib.hipcount_names.restype = ctypes.c_char_p
        self.categories = lib.hipcount_names().decode().split(",")

    def count(self, fn, stream: int) -> dict:
        """Counts of the HIP calls `fn()` makes (any thread), with `stream` as the caller's."""
        self.lib.hipcount_set_stream(ctypes.c_void_p(stream))
        self.lib.hipcount_reset()
        self.lib.hipcount_arm(1)
        try:
            fn()
        finally:
            self.lib.hipcount_arm(0)
        buf = (ctypes.c_long * len(self.categories))()
        self.lib.hipcount_read(buf, len(self.categories))
        return dict(zip(self.categories, buf))


def load_counter(path: str | Path | None = None) -> Counter:
    """Load the counter into the global symbol scope.  Fails if the HIP runtime is already
    loaded: its callers would then be bound to the runtime and never reach the hooks."""
    p = Path(path) if path else LIB_DIR / LIBNAME
    if not p.exists():
        raise CallCountError(f"{p} is not built; run __graft_entry__.build() first")
    if hip_runtime_loaded():
        raise CallCountError("the HIP runtime is already loaded in this process; the counter "
                             "must be loaded first (run callcount.py as its own process)")
    return Counter(ctypes.CDLL(str(p), mode=ctypes.RTLD_GLOBAL))


# Launches per steady call of each entry point and path.
EXPECTED_LAUNCHES = {
    "pow_abs_sqrt_mean": 1, "leaky": 1, "reward_to_go": 1, "ppo_clip": 1, "ppo_clip_entropy": 1,
    "ppo_clip_entropy_noalloc": 1,  # its first call on a device adds the scratch clear
    "efficient_kan": 2,          # kan_pack + kan_fused (spline order 3)
    "efficient_kan_rowwise": 1,  # kan_rowwise (other spline orders)
    "fp8_linear": 1,
    "quantize_e4m3": 2,          # qz_amax + qz_cast (unaligned, or more chunks than fit at once)
    "quantize_e4m3_fused": 1,    # qz_fused (aligned, every chunk resident at once)
}


def workloads():
    """(name, entry point, expectation key, make_args) for every hidden and public case of
    the six ops, the entropy variant of ppo_clip (allocating and not), the row-wise
    efficient_kan path and the quantiser (aligned and unaligned)."""
    import torch
    from cob_amd import capi, inputs, tasks

    def drop_in(op, case, entropy=False):
        def make():
            inp = inputs.make_inputs(op, case)
            if entropy:
                inp = dict(inp)
                g = torch.Generator().manual_seed(case["seed"] + 1)
                inp["entropy"] = torch.rand(inp["B"], inp["T"], inp["H"], generator=g)
                inp["entropy_coef"] = 0.01
            args = capi.device_args(op, inp)
            if op == "ppo_clip":
                args["output"] = torch.empty(8 if entropy else 6, device="cuda")
            else:
                for name, (shape, dtype) in capi.output_shapes(op, inp).items():
                    args[name] = torch.empty(shape, dtype=dtype, device="cuda")
            return args
        return make

    def quant(n, off):
        def make():
            g = torch.Generator().manual_seed(n)
            xb = torch.randn(n + off, generator=g).to("cuda")
            qb = torch.empty(n + off, dtype=torch.uint8, device="cuda")
            return dict(x=xb[off:], n=n, q=qb[off:], scale=torch.empty(1, device="cuda"))
        return make

    out = []
    for op in tasks.OPS:
        for case in tasks.all_cases(op):
            key = op
            if op == "efficient_kan" and case.get("spline_order", 3) != 3:
                key = "efficient_kan_rowwise"
            out.append((f"{op}/{case['name']}", op, key, drop_in(op, case)))
            if op == "ppo_clip":
                out.append((f"ppo_clip_entropy/{case['name']}", "ppo_clip_entropy", "ppo_clip_entropy",
                            drop_in(op, case, entropy=True)))
                out.append((f"ppo_clip_entropy_noalloc/{case['name']}", "ppo_clip_entropy_noalloc",
                            "ppo_clip_entropy_noalloc", drop_in(op, case, entropy=True)))
    for order in (1, 2):
        case = dict(name=f"B64_I40_O24_order{order}", seed=70 + order, small=True, timed=False,
                    B=64, I=40, O=24, spline_order=order)
        out.append((f"efficient_kan/{case['name']}", "efficient_kan", "efficient_kan_rowwise",
                    drop_in("efficient_kan", case)))
    out.append(("quantize_e4m3/aligned_n1000003", "quantize_e4m3", "quantize_e4m3_fused", quant(1_000_003, 0)))
    # 4096 x 4096, the fused path's whole resident capacity: still one launch.
    out.append(("quantize_e4m3/aligned_n16777216", "quantize_e4m3", "quantize_e4m3_fused", quant(1 << 24, 0)))
    out.append(("quantize_e4m3/aligned_n67108864", "quantize_e4m3", "quantize_e4m3", quant(1 << 26, 0)))
    out.append(("quantize_e4m3/unaligned_n4099", "quantize_e4m3", "quantize_e4m3", quant(4099, 1)))
    return out


def measure(counter: Counter, calls: int = 3, only: str = "") -> dict:
    import torch
    from cob_amd import capi
    lib = capi.load()
    stream = torch.cuda.Stream()
    handle = stream.cuda_stream
    res = {}
    for name, entry, key, make in workloads():
        if only and only not in name:
            continue
        args = make()
        torch.cuda.synchronize()

        def one():
            capi.call(lib, entry, args, handle)

        def several():
            for _ in range(calls):
                capi.call(lib, entry, args, handle)

        first = counter.count(one, handle)
        steady = counter.count(several, handle)
        torch.cuda.synchronize()
        res[name] = {"entry": capi.ENTRY[entry][0], "expect_launches": EXPECTED_LAUNCHES[key],
                     "first": first, "per_call": {k: v / calls for k, v in steady.items()}}
        print(f"[callcount] {name}: first {first}, per call {res[name]['per_call']}", file=sys.stderr, flush=True)
        del args
    return res


def table(res: dict, categories: list[str]) -> str:
    lines = ["| workload | entry point | " + " | ".join(categories) + " | first call: alloc, launch |",
             "|---|---|" + "---:|" * len(categories) + "---|"]
    for name, r in res.items():
        pc = r["per_call"]
        lines.append(f"| {name} | `{r['entry']}` | " + " | ".join(f"{pc[c]:g}" for c in categories)
                     + f" | {r['first']['alloc']}, {r['first']['launch']} |")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--json", help="write the counts as JSON here")
    ap.add_argument("--calls", type=int, default=3, help="steady calls averaged per workload")
    ap.add_argument("--only", default="", help="only workloads whose name contains this")
    a = ap.parse_args(argv)
    counter = load_counter()
    import torch
    if not torch.cuda.is_available():
        print("callcount.py needs a GPU", file=sys.stderr)
        return 1
    res = measure(counter, a.calls, a.only)
    if a.json:
        Path(a.json).write_text(json.dumps({"categories": counter.categories, "workloads": res}, indent=1))
    print(table(res, counter.categories))
    return 0


if __name__ == "__main__":
    sys.exit(main())
