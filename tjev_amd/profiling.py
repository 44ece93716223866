"""Summaries of rocprofv3 runs over bench.py, per kernel of the GDN library.

    python -m tjev_amd.profiling copy-probe [--mib 1024] [--reps 5]
        A plain device copy of known size (one elementwise kernel reading and writing --mib MiB
        per launch): what FETCH_SIZE / WRITE_SIZE read for it calibrates those counters.
    python -m tjev_amd.profiling stats --trace DIR --out FILE.md --command "..."
        Per-kernel launch counts and average durations from a --kernel-trace run (CSV output).
    python -m tjev_amd.profiling counters DIR [DIR ...] [--out FILE.md]
        Per-kernel averages of every counter of some --pmc runs.
    python -m tjev_amd.profiling mfma --pmc DIR --trace DIR --out FILE.md [--cus 256] [--xcds 8]
        MFMA work and busy fraction per kernel from one --pmc run of SQ_INSTS_VALU_MFMA_MOPS_BF16,
        SQ_INSTS_VALU_MFMA_MOPS_F32, SQ_VALU_MFMA_BUSY_CYCLES, SQ_BUSY_CYCLES and GRBM_GUI_ACTIVE,
        with the durations of a --kernel-trace run of the same command.
    python -m tjev_amd.profiling traffic --fetch DIR --write DIR --copy-fetch DIR --copy-write DIR
                                         --copy-mib 1024 --out FILE.json --command "..."
        HBM bytes per launch of every kernel from two --pmc runs (FETCH_SIZE, then WRITE_SIZE),
        each scaled by the copy probe's bytes / counter reading.

rocprofv3 names kernels by their symbols; the library's launch order per step (forward:
prep, chunk<0>, scan_fwd, out; backward: prep, chunk<1>, bwd_local, scan_bwd, bwd_grads, post,
reduce) maps them to the library's kernel names, k_prep's two launches alternating forward /
backward.
"""

from __future__ import annotations

import argparse
import csv
import json
import re
import statistics
import sys
from collections import defaultdict
from pathlib import Path

_FIXED = [("k_scan_fwd<", "gdn_scan_fwd"), ("k_scan_fwd_split<", "gdn_scan_fwd"), ("k_out<", "gdn_out"), ("k_bwd_local<", "gdn_bwd_local"),
          ("k_scan_bwd<", "gdn_scan_bwd"), ("k_bwd_grads<", "gdn_bwd_grads"), ("k_post<", "gdn_post"),
          ("k_reduce<", "gdn_reduce"), ("k_norm_fwd<", "gdn_norm_fwd"), ("k_norm_bwd<", "gdn_norm_bwd"),
          ("k_norm_reduce", "gdn_norm_reduce"), ("k_decode<", "gdn_decode"),
          ("k_final_state<", "gdn_final_state"), ("k_conv_state<", "gdn_conv_state")]


class _Namer:
    """Library kernel name of each dispatch, fed in dispatch order."""

    def __init__(self):
        self.preps = 0

    def __call__(self, symbol: str) -> str:
        for key, name in _FIXED:
            if key in symbol:
                return name
        if "k_prep<" in symbol:
            self.preps += 1
            return "gdn_prep_fwd" if self.preps % 2 else "gdn_prep_bwd"
        m = re.search(r"k_chunk<(?:[^,<>]+,\s*){4}(\d)\s*[,>]", symbol)
        if m:  # k_chunk<C, D, PI, PS, MODE, inverse form>: modes 0 and 2 run in the forward, 1 and 3 in the backward
            return "gdn_chunk_fwd" if m.group(1) in "02" else "gdn_chunk_bwd"
        return symbol


def _csvs(root: str, suffix: str) -> list[Path]:
    files = sorted(Path(root).rglob(f"*{suffix}"))
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {root} (run rocprofv3 with -f csv)")
    return files


def _rows(root: str, suffix: str) -> list[dict]:
    rows = []
    for f in _csvs(root, suffix):
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def trace_durations(root: str) -> dict[str, list[float]]:
    """Kernel durations in microseconds by library kernel name from kernel_trace.csv."""
    rows = sorted(_rows(root, "kernel_trace.csv"), key=lambda r: int(r.get("Dispatch_Id") or 0))
    name = _Namer()
    out: dict[str, list[float]] = defaultdict(list)
    for r in rows:
        out[name(r["Kernel_Name"])].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return out


def counter_per_dispatch(root: str, counter: str) -> dict[str, list[float]]:
    """Values of one counter per dispatch (summed over its dimensions), by library kernel name."""
    per: dict[int, list] = {}
    for r in _rows(root, "counter_collection.csv"):
        if r["Counter_Name"] != counter:
            continue
        d = int(r["Dispatch_Id"])
        if d not in per:
            per[d] = [r["Kernel_Name"], 0.0]
        per[d][1] += float(r["Counter_Value"])
    name = _Namer()
    out: dict[str, list[float]] = defaultdict(list)
    for d in sorted(per):
        out[name(per[d][0])].append(per[d][1])
    return out


def cmd_stats(args) -> int:
    dur = trace_durations(args.trace)
    rocprof_stats = _rows(args.trace, "kernel_stats.csv")
    lines = [f"# Kernel durations: {args.title}", "", "Command:", "", "```", args.command, "```", "",
             "Per library kernel, from kernel_trace.csv (k_prep's launches split forward / backward by order):", "",
             "| kernel | launches | avg us | min us | max us |", "|---|---:|---:|---:|---:|"]
    for k, v in sorted(dur.items(), key=lambda kv: -statistics.mean(kv[1])):
        lines.append(f"| {k} | {len(v)} | {statistics.mean(v):.1f} | {min(v):.1f} | {max(v):.1f} |")
    lines += ["", "rocprofv3 --stats (kernel_stats.csv) as written:", "",
              "| Name | Calls | AverageNs | Percentage |", "|---|---:|---:|---:|"]
    for r in rocprof_stats:
        lines.append(f"| {r.get('Name', '?')[:110]} | {r.get('Calls')} | {float(r.get('AverageNs', 0)):.0f} | "
                     f"{float(r.get('Percentage', 0)):.2f} |")
    Path(args.out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines[10:10 + len(dur) + 2]))
    return 0


def cmd_traffic(args) -> int:
    copy_bytes = args.copy_mib * 2 ** 20
    cf = [v for vs in counter_per_dispatch(args.copy_fetch, "FETCH_SIZE").values() for v in vs]
    cw = [v for vs in counter_per_dispatch(args.copy_write, "WRITE_SIZE").values() for v in vs]
    # the counters read KiB; the factor turns a reading into bytes
    f_fetch = copy_bytes / statistics.median(cf)
    f_write = copy_bytes / statistics.median(cw)
    fetch = counter_per_dispatch(args.fetch, "FETCH_SIZE")
    write = counter_per_dispatch(args.write, "WRITE_SIZE")
    kernels = {}
    for k in sorted(k for k in set(fetch) & set(write) if k.startswith("gdn_")):
        fk, wk = statistics.mean(fetch[k]), statistics.mean(write[k])
        kernels[k] = {"fetch_kib": fk, "write_kib": wk, "launches": len(fetch[k]),
                      "bytes": fk * f_fetch + wk * f_write}
    report = {"title": args.title, "command": args.command,
              "copy_probe": {"bytes_per_launch": copy_bytes, "fetch_kib": statistics.median(cf),
                             "write_kib": statistics.median(cw), "fetch_factor": f_fetch,
                             "write_factor": f_write},
              "kernels": kernels}
    Path(args.out).write_text(json.dumps(report, indent=1) + "\n")
    print(f"copy probe: FETCH {statistics.median(cf):.0f} KiB, WRITE {statistics.median(cw):.0f} KiB for "
          f"{copy_bytes} B -> factors {f_fetch:.1f}, {f_write:.1f} B per unit")
    for k, v in kernels.items():
        print(f"  {k:14s} fetch {v['fetch_kib']:12.0f} KiB  write {v['write_kib']:12.0f} KiB  "
              f"-> {v['bytes'] / 1e6:10.1f} MB")
    return 0


def cmd_counters(args) -> int:
    """Per library kernel, the average per dispatch of every counter in the --pmc runs."""
    table: dict[str, dict[str, float]] = defaultdict(dict)
    names: list[str] = []
    for root in args.runs:
        rows = _rows(root, "counter_collection.csv")
        for counter in sorted({r["Counter_Name"] for r in rows}):
            names.append(counter)
            for k, v in counter_per_dispatch(root, counter).items():
                table[k][counter] = statistics.mean(v)
    kernels = [k for k in table if k.startswith("gdn_")]
    lines = [f"# Counters: {args.title}", "", "Command:", "", "```", args.command, "```", "",
             "Average per dispatch.", "", "| kernel | " + " | ".join(names) + " |",
             "|---|" + "---:|" * len(names)]
    for k in kernels:
        lines.append(f"| {k} | " + " | ".join(f"{table[k].get(n, float('nan')):.4g}" for n in names) + " |")
    text = "\n".join(lines) + "\n"
    if args.out:
        Path(args.out).write_text(text)
    print(text)
    return 0


MFMA_COUNTERS = ("SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_VALU_MFMA_MOPS_F32", "SQ_VALU_MFMA_BUSY_CYCLES",
                 "SQ_BUSY_CYCLES", "GRBM_GUI_ACTIVE")


def cmd_mfma(args) -> int:
    """Executed MFMA work (MOPS counters, 512 FLOPs per unit) over the traced duration against
    the dense peaks, and SQ_VALU_MFMA_BUSY_CYCLES over the SIMDs' cycles (GRBM_GUI_ACTIVE reads
    the sum over the XCDs: per-XCD cycles x CUs x 4 SIMDs). The clock is the per-XCD cycles
    over the traced duration."""
    dur = trace_durations(args.trace)
    cnt = {c: counter_per_dispatch(args.pmc, c) for c in MFMA_COUNTERS}
    lines = [f"# MFMA counters: {args.title}", "", "Commands:", "", "```", args.command, "```", "",
             "Per dispatch, averaged over a kernel's launches. `executed` = 512 x (MOPS_BF16 + MOPS_F32)",
             "FLOPs (bf16x3 counts its three passes); `exec frac` = executed FLOP/s against the dense peak",
             "(2.5 PFLOP/s bf16, 157.3 TFLOP/s fp32); `busy` = SQ_VALU_MFMA_BUSY_CYCLES /",
             f"(GRBM_GUI_ACTIVE / {args.xcds} XCDs x {args.cus} CUs x 4 SIMDs), the MFMA pipes' busy fraction at",
             "the clock the kernel ran at (`clock` = GRBM_GUI_ACTIVE / XCDs over the duration).", "",
             "| kernel | avg us | clock GHz | executed bf16 GFLOP | executed fp32 GFLOP | exec frac | busy | "
             + " | ".join(MFMA_COUNTERS) + " |", "|---|" + "---:|" * (6 + len(MFMA_COUNTERS))]
    for k in sorted((k for k in cnt["GRBM_GUI_ACTIVE"] if k.startswith("gdn_")), key=lambda k: k):
        avg = {c: statistics.mean(cnt[c][k]) if cnt[c].get(k) else float("nan") for c in MFMA_COUNTERS}
        us = statistics.mean(dur[k]) if dur.get(k) else float("nan")
        bf, f32 = 512 * avg["SQ_INSTS_VALU_MFMA_MOPS_BF16"], 512 * avg["SQ_INSTS_VALU_MFMA_MOPS_F32"]
        frac = (bf / 2.5e15 + f32 / 157.3e12) / (us * 1e-6)
        cycles = avg["GRBM_GUI_ACTIVE"] / args.xcds
        busy = avg["SQ_VALU_MFMA_BUSY_CYCLES"] / (cycles * args.cus * 4)
        lines.append(f"| {k} | {us:.1f} | {cycles / (us * 1e3):.2f} | {bf / 1e9:.2f} | {f32 / 1e9:.2f} | {frac:.3f} | "
                     f"{busy:.3f} | "
                     + " | ".join(f"{avg[c]:.4g}" for c in MFMA_COUNTERS) + " |")
    text = "\n".join(lines) + "\n"
    Path(args.out).write_text(text)
    print(text)
    return 0


def cmd_copy_probe(args) -> int:
    import torch

    n = args.mib * 2 ** 20 // 4
    x = torch.empty(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(args.reps):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    print(f"copy probe: {args.reps} launches of {args.mib} MiB read + {args.mib} MiB written", flush=True)
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    p = sub.add_parser("copy-probe")
    p.add_argument("--mib", type=int, default=1024)
    p.add_argument("--reps", type=int, default=5)
    p = sub.add_parser("stats")
    p.add_argument("--trace", required=True)
    p.add_argument("--out", required=True)
    p.add_argument("--title", default="")
    p.add_argument("--command", default="")
    p = sub.add_parser("traffic")
    for k in ("fetch", "write", "copy_fetch", "copy_write", "out"):
        p.add_argument("--" + k.replace("_", "-"), dest=k, required=True)
    p.add_argument("--copy-mib", type=int, default=1024)
    p.add_argument("--title", default="")
    p.add_argument("--command", default="")
    p = sub.add_parser("counters")
    p.add_argument("runs", nargs="+", help="rocprofv3 --pmc output directories (CSV)")
    p.add_argument("--out", default=None)
    p.add_argument("--title", default="")
    p.add_argument("--command", default="")
    p = sub.add_parser("mfma")
    p.add_argument("--pmc", required=True)
    p.add_argument("--trace", required=True)
    p.add_argument("--out", required=True)
    p.add_argument("--cus", type=int, default=256)
    p.add_argument("--xcds", type=int, default=8)
    p.add_argument("--title", default="")
    p.add_argument("--command", default="")
    args = ap.parse_args(argv)
    return {"copy-probe": cmd_copy_probe, "stats": cmd_stats, "traffic": cmd_traffic,
            "counters": cmd_counters, "mfma": cmd_mfma}[args.cmd](args)


if __name__ == "__main__":
    sys.exit(main())
