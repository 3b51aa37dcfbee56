"""Summarise rocprofv3 CSV output of bench.py into the text kept under profiles/.

    python -m spq4k.rocprof_summary --trace DIR --fetch DIR --write DIR \
        --fetch-copy DIR --write-copy DIR --out profiles/NAME.md --json profiles/NAME.json

    python -m spq4k.rocprof_summary --stats DIR --out profiles/NAME.md --title T --command CMD

The second form turns the kernel_stats.csv of a `rocprofv3 --kernel-trace
--stats --output-format csv` run into a per-kernel table (calls, average,
minimum and maximum duration, share of GPU time).

--trace holds a `rocprofv3 --kernel-trace --stats --output-format csv` run of
`bench.py --no-cpu` (decode8b); --fetch / --write hold `--pmc FETCH_SIZE` /
`--pmc WRITE_SIZE` runs of the same command; --fetch-copy / --write-copy the
same two counters over `bench.py --config copy` (three 1 GiB device-to-device
copies), which scale the counters to bytes: factor = copied bytes / counter
bytes. Per decode stage the summary gives the average launch duration, the
HBM bytes read and written per launch (scaled) and the algorithmic bytes.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import shlex
import statistics
import sys

# The 8B decode step (bench.py build_decode8b): 36 x [qkv, o, gate_up, down], lm_head.
STAGES = ["qkv", "o", "gate_up", "down"]
SHAPES = {  # (rows, K) per matrix of each stage
    "qkv": [(4096, 4096), (1024, 4096), (1024, 4096)],
    "o": [(4096, 4096)],
    "gate_up": [(12288, 4096), (12288, 4096)],
    "down": [(4096, 12288)],
    "lm_head": [(151936, 4096)],
}
COPY_BYTES = 1 << 30


def alg_bytes(stage):
    return sum(M * (K // 256) * 144 + 4 * K + 4 * M for M, K in SHAPES[stage])


def _csv(d, suffix):
    files = glob.glob(os.path.join(d, f"*{suffix}")) or glob.glob(os.path.join(d, "**", f"*{suffix}"),
                                                                 recursive=True)
    if not files:
        raise FileNotFoundError(f"no *{suffix} in {d}")
    files.sort(key=os.path.getmtime)          # a directory reused across runs: the latest run's file
    with open(files[-1]) as f:
        return list(csv.DictReader(f))


def _gemv(rows):
    return [r for r in rows if "gemv" in r["Kernel_Name"]]


def _staged(rows, key):
    """Group the GEMV dispatches of the step replays by decode stage. The
    first 145 dispatches (in dispatch order) are one decode step, [qkv, o,
    gate_up, down] x 36 then lm_head; every following block of 145 whose
    kernel names repeat that sequence is another replay of the step, its
    dispatches mapped to stages by position (two stages may run the same
    kernel instantiation). Dispatches after the last such block (the
    per-stage replays) are left out."""
    rows = sorted(rows, key=lambda r: int(r[key]))
    pattern = [r["Kernel_Name"] for r in rows[:145]]
    if len(pattern) < 145:
        raise ValueError(f"{len(pattern)} GEMV dispatches: fewer than one decode step")
    out = {s: [] for s in STAGES + ["lm_head"]}
    for b in range(0, len(rows) - 144, 145):
        block = rows[b:b + 145]
        if [r["Kernel_Name"] for r in block] != pattern:
            break
        for i, r in enumerate(block):
            out["lm_head" if i == 144 else STAGES[i % 4]].append(r)
    return out


def _copy_factor(d):
    vals = [float(r["Counter_Value"]) * 1024 for r in _csv(d, "counter_collection.csv")
            if "copyBuffer" in r["Kernel_Name"]]
    return COPY_BYTES / statistics.median(vals), statistics.median(vals)


def stats_table(d, out, title, commands):
    """Per (kernel, grid) launch statistics from the kernel trace, in order of
    first dispatch (the trace keeps launches of one kernel at different sizes
    apart, which the stats file merges)."""
    trace = _csv(d, "kernel_trace.csv")
    key_id = "Dispatch_Id" if "Dispatch_Id" in trace[0] else "Start_Timestamp"
    trace.sort(key=lambda r: int(r[key_id]))
    groups = {}
    for r in trace:
        k = (r["Kernel_Name"], r.get("Grid_Size", r.get("Grid_Size_X", "")), r.get("Workgroup_Size",
                                                                                   r.get("Workgroup_Size_X", "")))
        groups.setdefault(k, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in groups.values())
    with open(out, "w") as f:
        f.write(f"# {title}\n\nCommands (from the repository root on the GPU box):\n\n```\n")
        for c in commands:
            f.write(c + "\n")
        f.write("```\n\nPer kernel and grid (threads), in order of first launch: durations from the kernel trace.\n\n"
                "| kernel | grid | wg | launches | avg us | min us | max us | % of GPU time |\n"
                "|---|---|---|---|---|---|---|---|\n")
        for (name, grid, wg), v in groups.items():
            name = name.replace("spq4k::", "").replace("(spq4k::GemmParams)", "").replace(
                "(spq4k::MoeParams)", "").replace("(spq4k::MoeFusedParams)", "").replace("(spq4k::GemvParams)", "")
            name = name.replace("(anonymous namespace)::", "")
            if "(" in name:
                name = name[:name.index("(")]
            f.write(f"| `{name}` | {grid} | {wg} | {len(v)} | {statistics.mean(v):.2f} | {min(v):.2f} | "
                    f"{max(v):.2f} | {100 * sum(v) / total:.1f} |\n")
    print(open(out).read())


def _own_command(argv):
    """The summary's own command line, recorded when no --command is given, so
    that the commands block never comes out empty (the profiler run that made
    the input is named with --command)."""
    return "PYTHONPATH=shannon-prime-burnhard_amd python3 -m spq4k.rocprof_summary " + shlex.join(argv)


def main(argv=None):
    if argv is None:
        argv = sys.argv[1:]
    if "--stats" in argv:
        ap = argparse.ArgumentParser()
        ap.add_argument("--stats", required=True)
        ap.add_argument("--out", required=True)
        ap.add_argument("--title", required=True)
        ap.add_argument("--command", action="append", default=[])
        a = ap.parse_args(argv)
        stats_table(a.stats, a.out, a.title, a.command or [_own_command(argv)])
        return 0
    ap = argparse.ArgumentParser()
    for a in ("trace", "fetch", "write", "fetch_copy", "write_copy", "out", "json"):
        ap.add_argument("--" + a.replace("_", "-"), required=True)
    ap.add_argument("--command", action="append", default=[], help="command line to record (repeatable)")
    args = ap.parse_args(argv)
    if not args.command:
        args.command = [_own_command(argv)]

    trace = _gemv(_csv(args.trace, "kernel_trace.csv"))
    by_stage = _staged(trace, "Dispatch_Id" if "Dispatch_Id" in trace[0] else "Start_Timestamp")
    f_fetch, copy_fetch = _copy_factor(args.fetch_copy)
    f_write, copy_write = _copy_factor(args.write_copy)
    fetch = _staged(_gemv(_csv(args.fetch, "counter_collection.csv")), "Dispatch_Id")
    write = _staged(_gemv(_csv(args.write, "counter_collection.csv")), "Dispatch_Id")

    lines = []
    tot_us = tot_alg = tot_hbm = 0.0
    n_launch = 0
    res = {"copy_calibration": {"bytes": COPY_BYTES, "fetch_counter_bytes": copy_fetch, "fetch_factor": f_fetch,
                                "write_counter_bytes": copy_write, "write_factor": f_write}, "stages": {}}
    for st in STAGES + ["lm_head"]:
        rs = by_stage[st]
        dur = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000 for r in rs]
        fb = [float(r["Counter_Value"]) * 1024 * f_fetch for r in fetch[st]]
        wb = [float(r["Counter_Value"]) * 1024 * f_write for r in write[st]]
        us = statistics.mean(dur)
        rd, wr = statistics.mean(fb), statistics.mean(wb)
        a = alg_bytes(st)
        per_step = 1 if st == "lm_head" else 36
        tot_us += us * per_step
        tot_alg += a * per_step
        tot_hbm += (rd + wr) * per_step
        n_launch += per_step
        kname = rs[0]["Kernel_Name"].replace("spq4k::", "").replace("(spq4k::GemvParams)", "")
        res["stages"][st] = {"kernel": kname, "launches_measured": len(dur), "avg_us": us, "hbm_read_bytes": rd,
                             "hbm_write_bytes": wr, "algorithmic_bytes": a}
        lines.append(f"| {st} | `{kname}` | {len(dur)} | {us:.3f} | {a / 1e6:.3f} | {rd / 1e6:.3f} | {wr / 1e6:.4f} "
                     f"| {(rd + wr) / a:.3f} | {a / us / 1e3:.0f} |")
    avg_us = tot_us / n_launch
    res["step"] = {"launches": n_launch, "sum_of_avg_launch_us": tot_us, "avg_launch_us": avg_us,
                   "algorithmic_bytes_per_launch": tot_alg / n_launch, "bytes_per_launch": tot_hbm / n_launch,
                   "hbm_over_algorithmic": tot_hbm / tot_alg, "achieved_GBps": tot_alg / tot_us / 1e3}
    with open(args.json, "w") as f:
        json.dump(res, f, indent=1)
    with open(args.out, "w") as f:
        f.write("# gemv_decode_kernel — 8B decode sweep (bench.py decode8b), rocprofv3 on MI355X\n\n")
        f.write("Commands (from the repository root on the GPU box):\n\n```\n")
        for c in args.command:
            f.write(c + "\n")
        f.write("```\n\n")
        f.write("Per stage: average launch duration from the kernel trace over the step replays; HBM bytes per launch from FETCH_SIZE / "
                "WRITE_SIZE (KiB per dispatch) scaled by the copy calibration below; algorithmic bytes = Q4_K "
                "weights + fp32 x + fp32 y of the launch.\n\n")
        f.write("| stage | kernel | launches | avg us | algorithmic MB | HBM read MB | HBM write MB | HBM/alg | "
                "alg GB/s |\n|---|---|---|---|---|---|---|---|---|\n")
        f.write("\n".join(lines) + "\n\n")
        f.write(f"Step: {n_launch} launches, sum of average durations {tot_us:.1f} us, average launch "
                f"{avg_us:.3f} us, algorithmic {tot_alg / n_launch / 1e6:.3f} MB/launch, HBM "
                f"{tot_hbm / n_launch / 1e6:.3f} MB/launch ({tot_hbm / tot_alg:.3f} x algorithmic), "
                f"{tot_alg / tot_us / 1e3:.1f} GB/s algorithmic.\n\n")
        f.write(f"Copy calibration: a {COPY_BYTES} B device-to-device copy reads {copy_fetch:.0f} B by FETCH_SIZE "
                f"(factor {f_fetch:.4f}) and writes {copy_write:.0f} B by WRITE_SIZE (factor {f_write:.4f}).\n")
    print(open(args.out).read())
    return 0


if __name__ == "__main__":
    sys.exit(main())
