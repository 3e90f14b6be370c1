"""ctypes binding of libtaskops.so (the C ABI declared in include/taskops.h).

`load()` opens the in-tree library and fails loudly when it is missing: there is no CPU
or PyTorch fallback behind these entry points.  `call(lib, op, args, stream)` invokes one
entry point on device tensors; `run_op(lib, op, inp)` is the convenience used by tests:
copy CPU inputs to the device, allocate outputs, call, synchronise, return the outputs.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

from . import LIB_DIR
from .tasks import load_task

LIBNAME = "libtaskops.so"

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float

# Entry point -> (argument names in C order, ctypes types).  Pointers are device pointers.
ENTRY = {
    "pow_abs_sqrt_mean": ("taskops_pow_abs_sqrt_mean",
                          [("inp", _P), ("target", _P), ("batch_size", _I64), ("height", _I64),
                           ("width", _I64), ("output", _P)]),
    "leaky": ("taskops_leaky",
              [("input_current", _P), ("mem0", _P), ("beta", _P), ("threshold", _P), ("T", _I32),
               ("B", _I32), ("H", _I32), ("spikes", _P), ("final_mem", _P)]),
    "reward_to_go": ("taskops_reward_to_go",
                     [("reward", _P), ("done", _P), ("gamma", _F32), ("B", _I32), ("T", _I32),
                      ("output", _P)]),
    "ppo_clip": ("taskops_ppo_clip",
                 [("B", _I32), ("T", _I32), ("H", _I32), ("current_log_prob", _P),
                  ("old_log_prob", _P), ("advantage", _P), ("clip_epsilon", _F32),
                  ("output", _P)]),
    "ppo_clip_entropy": ("taskops_ppo_clip_entropy",
                         [("B", _I32), ("T", _I32), ("H", _I32), ("current_log_prob", _P),
                          ("old_log_prob", _P), ("advantage", _P), ("entropy", _P),
                          ("clip_epsilon", _F32), ("entropy_coef", _F32), ("output", _P)]),
    # ppo_clip_entropy with its scratch in a fixed device array: no allocation at all.
    "ppo_clip_entropy_noalloc": ("taskops_ppo_clip_entropy_noalloc",
                                 [("B", _I32), ("T", _I32), ("H", _I32), ("current_log_prob", _P),
                                  ("old_log_prob", _P), ("advantage", _P), ("entropy", _P),
                                  ("clip_epsilon", _F32), ("entropy_coef", _F32), ("output", _P)]),
    "efficient_kan": ("taskops_efficient_kan",
                      [("x", _P), ("grid", _P), ("base_weight", _P), ("spline_weight", _P),
                       ("spline_scaler", _P), ("grid_size", _I32), ("spline_order", _I32),
                       ("B", _I32), ("I", _I32), ("O", _I32), ("out", _P)]),
    "fp8_linear": ("taskops_fp8_linear",
                   [("M", _I32), ("K", _I32), ("N", _I32), ("x_fp8", _P), ("scale_x", _F32),
                    ("w_fp8", _P), ("scale_w", _F32), ("bias", _P), ("output", _P)]),
    # Not a task op: the quantisation step before fp8_linear (reference.py:15-18).
    "quantize_e4m3": ("taskops_quantize_e4m3",
                      [("x", _P), ("n", _I64), ("q", _P), ("scale", _P)]),
}

EXPORTS = ["taskops_version"] + [v[0] for v in ENTRY.values()]

DTYPES = {"float32": torch.float32, "bfloat16": torch.bfloat16}


class TaskOpsError(RuntimeError):
    pass


def lib_path() -> Path:
    return LIB_DIR / LIBNAME


def load(path: str | Path | None = None) -> ctypes.CDLL:
    """Open libtaskops.so and declare every entry point's signature."""
    p = Path(path) if path else lib_path()
    if not p.exists():
        raise TaskOpsError(f"{p} is not built; run __graft_entry__.build() first "
                           "(there is no fallback path)")
    lib = ctypes.CDLL(str(p))
    lib.taskops_version.restype = ctypes.c_int
    lib.taskops_version.argtypes = []
    for op, (sym, params) in ENTRY.items():
        fn = getattr(lib, sym)
        fn.restype = ctypes.c_int
        fn.argtypes = [t for _, t in params] + [_P]
    return lib


def _ptr(t: torch.Tensor) -> int:
    if not t.is_cuda:
        raise TaskOpsError("taskops entry points take device tensors")
    if not t.is_contiguous():
        raise TaskOpsError("taskops entry points take contiguous tensors")
    return t.data_ptr()


def call(lib: ctypes.CDLL, op: str, args: dict, stream: int | None = None) -> None:
    """Call one entry point.  `args` maps C argument names to device tensors (pointers)
    or Python numbers (scalars).  `stream` is a raw hipStream_t handle (default: torch's
    current stream).  Raises TaskOpsError on a non-zero hipError_t."""
    sym, params = ENTRY[op]
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    cargs = []
    for name, ctype in params:
        v = args[name]
        cargs.append(ctypes.c_void_p(_ptr(v)) if ctype is _P else ctype(v))
    rc = getattr(lib, sym)(*cargs, ctypes.c_void_p(stream))
    if rc != 0:
        raise TaskOpsError(f"{sym} returned hipError_t {rc}")


def bind(lib: ctypes.CDLL, op: str, args: dict, stream: int | None = None):
    """`call` with the arguments converted once: returns a function of no arguments that
    invokes the entry point and raises TaskOpsError on a non-zero hipError_t.  The tensors
    in `args` must stay alive (and at the same addresses) while it is used."""
    sym, params = ENTRY[op]
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    cargs = tuple(ctypes.c_void_p(_ptr(args[name])) if ctype is _P else ctype(args[name])
                  for name, ctype in params) + (ctypes.c_void_p(stream),)
    fn = getattr(lib, sym)

    def run() -> None:
        rc = fn(*cargs)
        if rc != 0:
            raise TaskOpsError(f"{sym} returned hipError_t {rc}")
    return run


def output_shapes(op: str, inp: dict) -> dict:
    """Output name -> (shape, dtype) for the drop-in ops (from the task spec)."""
    task = load_task(op)
    env = {k: v for k, v in inp.items() if not isinstance(v, torch.Tensor)}
    out = {}
    for name, o in task["outputs"].items():
        shape = [int(eval(str(s), {}, env)) for s in o["shape"]]
        out[name] = (shape, DTYPES[o["dtype"]])
    return out


def device_args(op: str, inp: dict, device="cuda") -> dict:
    """Inputs on the device; fp8 tensors are viewed as the C ABI's raw bytes (bf16 and
    bool tensors already have the raw layout the C ABI expects)."""
    res = {}
    for k, v in inp.items():
        if isinstance(v, torch.Tensor):
            t = v.contiguous()
            if t.dtype == torch.float8_e4m3fn:
                t = t.view(torch.uint8)
            res[k] = t.to(device)
        else:
            res[k] = v
    return res


def run_op(lib: ctypes.CDLL, op: str, inp: dict, entropy: bool | None = None) -> dict:
    """Run `op` on CPU inputs `inp`; return its outputs as device tensors (synchronised).
    For ppo_clip, inputs holding `entropy` run the 8-output entropy entry point."""
    args = device_args(op, inp)
    if op == "ppo_clip" and (entropy if entropy is not None else "entropy" in inp):
        out = torch.full((8,), float("nan"), device="cuda")
        args["output"] = out
        call(lib, "ppo_clip_entropy", args)
        torch.cuda.synchronize()
        return {"output": out}
    outs = {}
    for name, (shape, dtype) in output_shapes(op, inp).items():
        outs[name] = torch.full(shape, float("nan"), dtype=dtype, device="cuda")
        args[name] = outs[name]
    call(lib, op, args)
    torch.cuda.synchronize()
    return outs
