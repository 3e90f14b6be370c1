"""Summaries of rocprofv3 result databases, for the text files kept under profiles/.

    python cuda-optimization-benchmark_amd/profiling.py stats DIR
        Per-kernel dispatch count and average / median / min / max duration from a
        `rocprofv3 --kernel-trace --stats -d DIR` run (a markdown table).

    python cuda-optimization-benchmark_amd/profiling.py mfma DIR [--simds 1024] [--xcds 8] [--json OUT]
        MFMA utilisation per kernel from a `rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES
        SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_VALU_MFMA_MOPS_F8 GRBM_GUI_ACTIVE` run:
        busy = MFMA-busy cycles summed over SIMDs / (GUI-active cycles x SIMDs), the
        MfmaUtil expression of rocprofiler's counter definitions, and the MFMA work
        executed per dispatch (MOPS x 512 FLOP).  The result database holds each counter
        summed over its instances; GRBM_GUI_ACTIVE has one instance per XCD, all counting
        the same cycles (MfmaUtil takes their maximum), so the sum is divided by the XCDs.

    python cuda-optimization-benchmark_amd/profiling.py traffic FETCH_DIR WRITE_DIR [--json OUT]
        Per-kernel HBM traffic per dispatch from two `rocprofv3 --pmc FETCH_SIZE` and
        `--pmc WRITE_SIZE` runs of `bench.py --copy-probe`.  Both counters (KiB per
        dispatch) are scaled by what they read for the probe's plain device copy of
        bench.COPY_PROBE_BYTES, so a copy of n bytes reads exactly n fetched and n written.
        With --json, writes {"values": {bench op key: bytes per launch of its dominant
        kernel}, "call_values": {op: bytes per call, every kernel}, "source", "commit"}.

Only the standard library is used: the databases are SQLite files.
"""
from __future__ import annotations

import argparse
import collections
import glob
import json
import sqlite3
import statistics
import sys

# Dominant kernel of each bench workload (a substring of the mangled kernel name); a
# tuple names the kernels one call launches, whose traffic is summed.
DOMINANT = {
    "reward_to_go": "reward_to_go_kernel",
    "pow_abs_sqrt_mean": "pow_abs_sqrt_mean_kernel",
    "leaky": "leaky_kernel",
    # <threads, unroll, vector loads, entropy, nt>: the entropy and the drop-in variants
    "ppo_clip": "ppo_clip_kernel<512, 2, true, true,",
    "ppo_clip_dropin": "ppo_clip_kernel<512, 2, true, false,",
    "efficient_kan": "kan_fused",
    "fp8_linear": "fp8_gemm_wide",
    "fp8_linear_m16": "fp8_gemm_skinny_flat",
    "fp8_linear_timed": "fp8_gemm_half",
    "quantize_e4m3": "qz_fused",
}
# Every kernel one call launches, for the ops that launch more than one; their traffic is
# summed into the call's total.
CALL_KERNELS = {
    "efficient_kan": ("kan_pack", "kan_fused"),
}
COPY_PROBE_BYTES = 256 << 20


def _db(d: str) -> sqlite3.Connection:
    files = sorted(glob.glob(f"{d}/**/*results.db", recursive=True))
    if not files:
        raise SystemExit(f"no *results.db under {d}")
    return sqlite3.connect(files[0])


def kernel_stats(d: str) -> dict:
    c = _db(d)
    agg = collections.defaultdict(list)
    for name, dur in c.execute("select name, duration from kernels"):
        agg[name].append(dur / 1e3)
    return agg


def _short(name: str, width: int = 72) -> str:
    return name if len(name) <= width else name[: width - 3] + "..."


def print_stats(d: str) -> None:
    agg = kernel_stats(d)
    print("| kernel | calls | avg us | median us | min us | max us |")
    print("|---|---:|---:|---:|---:|---:|")
    for k, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{_short(k)}` | {len(v)} | {statistics.mean(v):.2f} | {statistics.median(v):.2f} "
              f"| {min(v):.2f} | {max(v):.2f} |")


def counter_values(d: str, counter: str, reduce: str = "sum") -> dict:
    """kernel name -> per-dispatch counter values (summed, or with reduce="max" the
    largest, over the counter's instances), in dispatch order."""
    c = _db(d)
    per = collections.defaultdict(float)
    names = {}
    for name, disp, val in c.execute(
            "select kernel_name, dispatch_id, value from counters_collection where counter_name = ?",
            (counter,)):
        per[disp] = max(per[disp], val) if reduce == "max" else per[disp] + val
        names[disp] = name
    agg = collections.defaultdict(list)
    for disp in sorted(per):
        agg[names[disp]].append(per[disp])
    return agg


def _copy_calibration(vals: dict) -> tuple[str, float]:
    """The probe's copies: the three largest dispatches of a copy kernel (the probe's
    256 MiB copies are the largest copies in a bench run), which must agree within 1%."""
    cands = sorted(((v, k) for k, vs in vals.items() if "copy" in k.lower() for v in vs), reverse=True)
    if len(cands) < 3:
        raise SystemExit("no copy probe found: run bench.py with --copy-probe")
    top = [v for v, _ in cands[:3]]
    if max(top) > 1.01 * min(top):
        raise SystemExit(f"copy probe dispatches disagree: {top}")
    return cands[0][1], statistics.mean(top)


def traffic(fetch_dir: str, write_dir: str) -> dict:
    f = counter_values(fetch_dir, "FETCH_SIZE")
    w = counter_values(write_dir, "WRITE_SIZE")
    fk, fv = _copy_calibration(f)
    _, wv = _copy_calibration(w)
    ff = COPY_PROBE_BYTES / fv   # bytes per counter unit, from the copy
    wf = COPY_PROBE_BYTES / wv
    rows = {}
    for k in sorted(set(f) | set(w)):
        n = len(f.get(k) or w.get(k))
        rows[k] = {"dispatches": n,
                   "fetch_bytes": statistics.mean(f[k]) * ff if k in f else None,
                   "write_bytes": statistics.mean(w[k]) * wf if k in w else None}
    return {"copy_kernel": fk, "fetch_factor": ff, "write_factor": wf,
            "copy_fetch_kib": fv, "copy_write_kib": wv, "kernels": rows}


def print_traffic(t: dict) -> None:
    print(f"Calibration: `{_short(t['copy_kernel'])}` copying {COPY_PROBE_BYTES} bytes reads "
          f"FETCH_SIZE {t['copy_fetch_kib']:.1f} and WRITE_SIZE {t['copy_write_kib']:.1f} per dispatch; "
          f"factors {t['fetch_factor']:.2f} and {t['write_factor']:.2f} bytes per unit.\n")
    print("| kernel | dispatches | fetched MB / launch | written MB / launch | total MB |")
    print("|---|---:|---:|---:|---:|")
    for k, r in t["kernels"].items():
        fb, wb = r["fetch_bytes"] or 0.0, r["write_bytes"] or 0.0
        print(f"| `{_short(k)}` | {r['dispatches']} | {fb / 1e6:.2f} | {wb / 1e6:.2f} | {(fb + wb) / 1e6:.2f} |")


def dominant_traffic(t: dict, table: dict = DOMINANT) -> dict:
    out = {}
    for op, subs in table.items():
        total, found = 0.0, True
        for sub in (subs,) if isinstance(subs, str) else subs:
            hits = [r for k, r in t["kernels"].items() if sub in k and "copy" not in k.lower()]
            if not hits:
                found = False
                break
            total += statistics.mean(r["fetch_bytes"] or 0.0 for r in hits)
            total += statistics.mean(r["write_bytes"] or 0.0 for r in hits)
        if found:
            out[op] = int(round(total))
    return out


MI355X_SIMDS = 256 * 4
MI355X_XCDS = 8


def dispatch_durations(d: str) -> dict:
    """kernel name -> per-dispatch durations in ns, in dispatch order (the same dispatches
    counter_values returns)."""
    agg = collections.defaultdict(list)
    for name, _, dur in sorted(_db(d).execute("select name, dispatch_id, duration from kernels"),
                               key=lambda r: r[1]):
        agg[name].append(float(dur))
    return agg


def mfma_util(d: str, simds: int = MI355X_SIMDS, xcds: int = MI355X_XCDS) -> dict:
    """kernel -> {dispatches, busy_pct, f16_flop, f8_flop, clock_ghz} (means over dispatches).
    clock_ghz is GRBM_GUI_ACTIVE's cycles per XCD over the dispatch's duration: the shader
    clock the kernel ran at (the peaks are quoted at 2.4 GHz)."""
    busy = counter_values(d, "SQ_VALU_MFMA_BUSY_CYCLES")
    gui = {k: [v / xcds for v in vs] for k, vs in counter_values(d, "GRBM_GUI_ACTIVE").items()}
    f16 = counter_values(d, "SQ_INSTS_VALU_MFMA_MOPS_F16")
    f8 = counter_values(d, "SQ_INSTS_VALU_MFMA_MOPS_F8")
    durs = dispatch_durations(d)
    out = {}
    for k, b in busy.items():
        g = gui.get(k)
        if not g or sum(b) == 0:
            continue
        t = durs.get(k, [])
        clock = statistics.mean(gg / tt for gg, tt in zip(g, t) if tt > 0) if len(t) == len(g) else float("nan")
        out[k] = {"dispatches": len(b),
                  "busy_pct": 100.0 * statistics.mean(bb / (gg * simds) for bb, gg in zip(b, g)),
                  "f16_flop": 512.0 * statistics.mean(f16.get(k, [0.0])),
                  "f8_flop": 512.0 * statistics.mean(f8.get(k, [0.0])),
                  "clock_ghz": clock}
    return out


def print_mfma(u: dict) -> None:
    print("| kernel | dispatches | MFMA busy % | clock GHz | fp16 MFMA FLOP / dispatch | fp8 MFMA FLOP / dispatch |")
    print("|---|---:|---:|---:|---:|---:|")
    for k, r in sorted(u.items(), key=lambda kv: -kv[1]["busy_pct"]):
        print(f"| `{_short(k)}` | {r['dispatches']} | {r['busy_pct']:.1f} | {r['clock_ghz']:.2f} | "
              f"{r['f16_flop']:.4g} | {r['f8_flop']:.4g} |")


def _write_json(path: str, body: dict, a) -> None:
    """The summary bench.py reads: the figures plus where they came from (the profiles/
    file that shows them and the commit of the profiled build)."""
    body = dict(body, source=a.source, commit=a.commit)
    with open(path, "w") as fh:
        json.dump(body, fh, indent=1, sort_keys=True)
        fh.write("\n")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    m = sub.add_parser("mfma")
    m.add_argument("dir")
    m.add_argument("--simds", type=int, default=MI355X_SIMDS)
    m.add_argument("--xcds", type=int, default=MI355X_XCDS)
    m.add_argument("--json", help="write {bench op key: MFMA busy %% of its dominant kernel}")
    c = sub.add_parser("counters", help="mean of each named counter per dispatch, for kernels matching --kernel")
    c.add_argument("dir")
    c.add_argument("names", nargs="+")
    c.add_argument("--kernel", default="", help="substring of the kernel names to show")
    t = sub.add_parser("traffic")
    t.add_argument("fetch_dir")
    t.add_argument("write_dir")
    t.add_argument("--json")
    for p in (m, t):
        p.add_argument("--commit", default="", help="the source commit the profiled build came from")
        p.add_argument("--source", default="", help="the profiles/ summary these figures appear in")
    a = ap.parse_args(argv)
    if a.cmd == "stats":
        print_stats(a.dir)
    elif a.cmd == "counters":
        print("| counter | kernel | dispatches | mean per dispatch |")
        print("|---|---|---:|---:|")
        for name in a.names:
            for k, vs in sorted(counter_values(a.dir, name).items()):
                if a.kernel in k and vs:
                    print(f"| {name} | `{_short(k, 48)}` | {len(vs)} | {statistics.mean(vs):.4g} |")
    elif a.cmd == "mfma":
        u = mfma_util(a.dir, a.simds, a.xcds)
        print_mfma(u)
        if a.json:
            dom = {}
            for op, sub in DOMINANT.items():
                hits = [r["busy_pct"] for k, r in u.items() if isinstance(sub, str) and sub in k]
                if hits:
                    dom[op] = round(statistics.mean(hits), 1)
            _write_json(a.json, {"values": dom}, a)
    else:
        tr = traffic(a.fetch_dir, a.write_dir)
        print_traffic(tr)
        if a.json:
            _write_json(a.json, {"values": dominant_traffic(tr),
                                 "call_values": dominant_traffic(tr, CALL_KERNELS)}, a)
    return 0


if __name__ == "__main__":
    sys.exit(main())
