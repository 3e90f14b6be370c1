"""The grading layer on the CPU: signature parsing and the shim text, argument packing, the
arena's layout and stray-write detection, the tolerance tally (against a scalar
restatement of the tasks' rule on random data), and the label rules with their order."""
import ctypes
import math
import struct

import numpy as np
import pytest
import torch

from cob_amd import tasks
from cob_amd.grader import signature
from cob_amd.grader.arena import ALIGN, GUARD_BYTES, GUARD_FILL, POISON_FILL, Arena
from cob_amd.grader.entry import pack
from cob_amd.grader.labels import LABELS, case_outcome, kernel_status
from cob_amd.grader.tolerance import tally


# -- signatures and the shim --------------------------------------------------------------
def test_six_tasks():
    assert sorted(tasks.OPS) == sorted(["pow_abs_sqrt_mean", "leaky", "efficient_kan", "fp8_linear",
                                        "ppo_clip", "reward_to_go"])


@pytest.mark.parametrize("op", tasks.OPS)
def test_task_signature(op):
    t = tasks.load_task(op)
    names = [p.name for p in t["params"]]
    assert len(set(names)) == len(names) and set(t["outputs"]) <= set(names)
    assert all(p.pointer and not p.ctype.startswith("const") for p in t["params"] if p.name in t["outputs"])
    assert all(p.ctype.startswith("const") for p in t["params"] if p.pointer and p.name not in t["outputs"])
    text = signature.shim(signature.parse(t["hip_signature"]))
    assert text.count("a[") == len(names) and 'extern "C" void grader_entry(void** a)' in text
    assert "__nv_" not in text
    assert sum(bool(c.get("small")) for c in t["cases"]) >= 1 and sum(bool(c.get("timed")) for c in t["cases"]) == 1


def test_parse_spacing_and_qualifiers():
    a = signature.parse("void reference(const float *x,const int64_t n , float*  out)")
    b = signature.parse("void reference(const float* x, const int64_t n, float *out);")
    assert a == b
    assert [(p.name, p.ctype, p.pointer, p.base, p.cell) for p in a] == [
        ("x", "const float*", True, "float", "const float*"),
        ("n", "const int64_t", False, "int64_t", "int64_t"),
        ("out", "float*", True, "float", "float*")]


def test_shim_text_for_mixed_types():
    ps = signature.parse("void reference(const int32_t M, const __hip_fp8_e4m3* q, float s, bool* flags, "
                         "__hip_bfloat16* y);")
    text = signature.shim(ps, header="k.hpp")
    assert text.splitlines()[0] == '#include "k.hpp"'
    assert ("reference(*(int32_t*)a[0], *(const __hip_fp8_e4m3**)a[1], *(float*)a[2], *(bool**)a[3], "
            "*(__hip_bfloat16**)a[4]);") in text


@pytest.mark.parametrize("bad", ["void f(int a);", "void reference(int *);"])
def test_parse_rejects(bad):
    with pytest.raises(ValueError):
        signature.parse(bad)


def test_pack_cells():
    ps = signature.parse("void reference(const int32_t M, const float* x, float g, int64_t n, double d, "
                         "bool b, float* out);")
    addrs = {"x": 0x1234_5678_9ABC, "out": 0xFFFF_0000_1111}
    cells, table = pack(ps, addrs.__getitem__, {"M": -7, "g": 0.99, "n": 1 << 40, "d": -2.5, "b": True})
    raw = bytes(cells)
    assert [table[i] - ctypes.addressof(cells) for i in range(len(ps))] == [8 * i for i in range(len(ps))]
    assert struct.unpack_from("<i", raw, 0)[0] == -7
    assert struct.unpack_from("<Q", raw, 8)[0] == addrs["x"]
    assert struct.unpack_from("<f", raw, 16)[0] == np.float32(0.99)
    assert struct.unpack_from("<q", raw, 24)[0] == 1 << 40
    assert struct.unpack_from("<d", raw, 32)[0] == -2.5
    assert raw[40] == 1
    assert struct.unpack_from("<Q", raw, 48)[0] == addrs["out"]


# -- the arena ----------------------------------------------------------------------------
def _arena():
    return Arena([("x", "in", torch.float32, [3, 5]), ("m", "in", torch.bool, [7]),
                  ("y", "out", torch.bfloat16, [9]), ("z", "out", torch.float32, [])], device="cpu")


def test_arena_layout():
    a = _arena()
    prev_end = 0
    for r in a.regions:
        assert r.start % ALIGN == 0 and r.start - prev_end >= GUARD_BYTES
        prev_end = r.start + r.nbytes
    assert a.size - prev_end >= GUARD_BYTES
    assert [r.nbytes for r in a.regions] == [60, 7, 18, 4]
    x = torch.arange(15, dtype=torch.float32).reshape(3, 5)
    m = torch.tensor([1, 0, 1, 1, 0, 0, 1], dtype=torch.bool)
    img = a.image({"x": x, "m": m})
    a.stage(img)
    assert torch.equal(a.view("x"), x) and torch.equal(a.view("m"), m)
    assert bool((a.view("y").view(torch.uint8) == POISON_FILL).all())
    for label, lo, hi in a.watched:
        if label.startswith("gap"):
            assert hi - lo >= GUARD_BYTES and bool((a.mem[lo:hi] == GUARD_FILL).all())
    assert a.strays() == []
    a.view("y").fill_(3.0)
    a.view("z").fill_(-1.0)
    assert a.strays() == []                       # outputs may change


@pytest.mark.parametrize("where,label", [
    (lambda a: a.by_name["x"].start - 1, "gap before x"),
    (lambda a: a.by_name["x"].start + 60, "gap before m"),     # between x and m
    (lambda a: a.by_name["y"].start + 18, "gap before z"),     # just past y
    (lambda a: a.size - 1, "gap after z"),
    (lambda a: a.by_name["m"].start + 6, "input m"),
])
def test_arena_strays(where, label):
    a = _arena()
    a.stage(a.image({"x": torch.zeros(3, 5), "m": torch.zeros(7, dtype=torch.bool)}))
    off = where(a)
    a.mem[off] ^= 0x5A
    assert a.strays() == [{"region": label, "first": off, "bytes": 1}]


# -- the tolerance tally ------------------------------------------------------------------
def _rule(got, want, atol, rtol):
    """The tasks' agreement rule for one element, written out case by case."""
    if math.isnan(want):
        return math.isnan(got)
    if math.isinf(want):
        return got == want
    if math.isnan(got) or math.isinf(got):
        return False
    return abs(got - want) <= atol + rtol * abs(want)


def test_tally_matches_scalar_rule():
    rng = np.random.default_rng(7)
    for trial in range(20):
        n = 400
        want = rng.normal(size=n) * 10.0 ** rng.integers(-3, 3)
        got = want + rng.normal(size=n) * 10.0 ** rng.integers(-6, 0)
        specials = [np.nan, np.inf, -np.inf, 0.0]
        for i in rng.choice(n, 30, replace=False):
            want[i] = rng.choice(specials)
        for i in rng.choice(n, 30, replace=False):
            got[i] = rng.choice(specials + [want[i]])
        atol, rtol = float(10 ** rng.uniform(-6, -1)), float(10 ** rng.uniform(-6, -1))
        t = tally(got, want, {"atol": atol, "rtol": rtol})
        bad = [i for i in range(n) if not _rule(got[i], want[i], atol, rtol)]
        assert t["mismatched"] == len(bad), trial
        assert (t["first"] or {}).get("index") == (bad[0] if bad else None)


def test_tally_bound_is_inclusive_and_worst_ratio():
    tol = {"atol": 0.5, "rtol": 0.25}                # bound at want = 2 is exactly 1.0
    assert tally(np.array([3.0]), np.array([2.0]), tol)["mismatched"] == 0
    assert tally(np.array([3.0]), np.array([2.0]), tol)["worst"] == 1.0
    assert tally(np.array([np.nextafter(3.0, 4.0)]), np.array([2.0]), tol)["mismatched"] == 1
    t = tally(np.array([4.5, 1.0]), np.array([4.0, 1.0]), {"atol": 0.0, "rtol": 0.25})
    assert t["worst"] == 0.5 and t["mismatched"] == 0 and t["first"] is None


def test_tally_unwritten_counts_only_filled_elements():
    want = np.array([1.0, 2.0, np.nan, 4.0])
    got = torch.tensor([1.0, 0.0, 0.0, 4.0])
    got.view(torch.uint8)[4:12] = POISON_FILL                 # elements 1 and 2 left at 0xFF
    t = tally(got, want, {"atol": 1e-6, "rtol": 0.0})
    # element 2 is NaN against a NaN reference: it agrees, so only element 1 counts
    assert (t["mismatched"], t["unwritten"], t["first"]["index"]) == (1, 1, 1)
    got[3] = 5.0                                             # a written but wrong element
    t = tally(got, want, {"atol": 1e-6, "rtol": 0.0})
    assert (t["mismatched"], t["unwritten"]) == (2, 1)


def test_tally_bf16_and_size():
    tol = {"atol": 0.0, "rtol": 2.0 ** -8}
    want = np.array([1.0, 3.0, -0.5])
    assert tally(torch.tensor(want, dtype=torch.bfloat16), want, tol)["mismatched"] == 0
    assert tally(torch.tensor([1.0, 3.0 + 2 ** -5, -0.5], dtype=torch.bfloat16), want, tol)["mismatched"] == 1
    t = tally(torch.zeros(3), np.zeros(4), tol)
    assert t["size_ok"] is False and t["mismatched"] == 4


# -- labels ---------------------------------------------------------------------------------
def _report(**change):
    ok = {"elements": 10, "size_ok": True, "mismatched": 0, "unwritten": 0, "worst": 0.1, "first": None}
    r = {"case": "c", "state": "finished", "repeat_identical": True,
         "calls": [{"call": n, "inputs": s, "strays": []} for n, s in ((1, "A"), (2, "B"), (3, "A"))],
         "checks": {"1": {"out": dict(ok)}, "2": {"out": dict(ok)}}}
    for path, v in change.items():
        node = r
        keys = path.split("__")
        for k in keys[:-1]:
            node = node[int(k)] if isinstance(node, list) else node[k]
        node[keys[-1]] = v
    return r


GAP = [{"region": "gap after out", "first": 9000, "bytes": 1}]
INP = [{"region": "input x", "first": 4096, "bytes": 2}]


@pytest.mark.parametrize("report,outcome,label,where", [
    (_report(), "pass", None, None),
    (_report(checks__1__out__mismatched=3), "fail", "wrong value", "call 1: out"),
    (_report(checks__1__out__mismatched=3, checks__1__out__unwritten=3), "fail", "unwritten output", "call 1: out"),
    (_report(checks__1__out__mismatched=3, checks__1__out__unwritten=2), "fail", "wrong value", "call 1: out"),
    (_report(checks__1__out__size_ok=False, checks__1__out__mismatched=10), "fail", "wrong shape", "call 1: out"),
    (_report(checks__2__out__mismatched=10), "fail", "stale state", "call 2: out"),
    (_report(calls__2__strays=GAP), "fail", "out-of-bounds write", "call 3: gap after out (byte 9000, 1 bytes)"),
    (_report(calls__1__strays=INP), "fail", "input modified", "call 2: input x (byte 4096, 2 bytes)"),
    (_report(state="crashed", calls__0__error="illegal address"), "fail", "cuda error", "call 1: illegal address"),
    (_report(state="crashed"), "fail", "crash", "crashed"),
    (_report(state="timeout"), "timeout", "timeout", "timeout"),
    (_report(state="not started", calls=[]), "grader_error", None, "before call 1"),
])
def test_case_labels(report, outcome, label, where):
    o = case_outcome(report)
    assert (o["outcome"], o["label"], o["where"]) == (outcome, label, where)


def test_label_precedence():
    """Calls are read one at a time, each with its checks in the order cuda error,
    out-of-bounds write, input modified, as graders/verdict.py:37-44 reads them: a change
    to an input on call 1 outranks a guard hit on call 2, and within one call the guard hit
    comes first.  Judged outputs are read one at a time, in output order."""
    assert LABELS.index("out-of-bounds write") < LABELS.index("input modified") < LABELS.index("wrong value")
    r = _report(calls__0__strays=INP, calls__1__strays=GAP, checks__1__out__mismatched=1)
    assert (case_outcome(r)["label"], case_outcome(r)["where"]) == ("input modified", "call 1: input x (byte 4096, 2 bytes)")
    r = _report(calls__1__strays=INP + GAP)
    assert case_outcome(r)["label"] == "out-of-bounds write"
    r = _report(calls__2__error="launch failure", calls__0__strays=GAP)
    assert case_outcome(r)["label"] == "out-of-bounds write"
    r = _report(checks__1__out__mismatched=1, checks__2__out__mismatched=1)
    assert case_outcome(r)["label"] == "wrong value"
    r = _report(checks__1__out__mismatched=2)
    r["checks"]["1"]["other"] = dict(r["checks"]["1"]["out"], size_ok=False, mismatched=10)
    assert (case_outcome(r)["label"], case_outcome(r)["where"]) == ("wrong value", "call 1: out")
    r["checks"]["1"]["out"]["mismatched"] = 0
    assert (case_outcome(r)["label"], case_outcome(r)["where"]) == ("wrong shape", "call 1: other")


def test_kernel_status_over_passes():
    good, bad = _report(), _report(checks__1__out__mismatched=1)
    lost = _report(state="not started", calls=[])
    assert kernel_status([[good, good], [good, good]])["status"] == "pass"
    st = kernel_status([[good, good], [good, bad]])
    assert (st["status"], st["label"], st["passes"]) == ("flip", "wrong value", ["pass", "fail"])
    st = kernel_status([[bad], [bad]])
    assert (st["status"], st["label"]) == ("fail", "wrong value")
    assert kernel_status([[good], [lost]])["status"] == "grader_error"
    assert kernel_status([])["status"] == "grader_error"
    assert kernel_status([[_report(repeat_identical=False)]])["repeat_identical"] is False
    st = kernel_status([[good, _report(case="second", checks__2__out__mismatched=4)]])
    assert (st["case"], st["label"]) == ("second", "stale state")
