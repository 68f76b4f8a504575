"""Kernel durations of the benchmark's timed legs, from a rocprofv3 kernel
trace of bench.py run with the driver's flags:

    rocprofv3 --kernel-trace --stats --output-format csv -d <run>/trace -o trace -- \\
        python3 bench.py --gpus 1 --steps 20 --warmup 5 > <run>/bench.json
    python3 -m dequant_project_amd.traces <run> [--counters <counter run>] [--out profiles/<name>.md]

The timed phase opens with the streaming-read ceiling leg (its warm-up and
timed launches of stream_read_kernel back to back); the other legs follow in
the order bench.py records (protocol.order), each replaying its graph
warm-up + steps times, launches_per_step dispatches per replay
(protocol.legs; a leg recorded without a count, such as the one mixing torch
ops into its step, ends the split). Only the timed replays are summarized.
With the counter
pass's output (dequant_project_amd.counters: <counter run>/FETCH_SIZE.json),
each launch also gets its algorithmic bytes, hence GB/s per kernel.

The --stats summary averages a kernel over every dispatch of the run
(eager capture passes, the launch-event pass, legs of other shapes); the
per-leg figures here are what the benchmark's numbers correspond to.
"""
import argparse
import csv
import gzip
import json
import os
import statistics
import sys
from collections import OrderedDict

PEAK_GBS = 8000.0
CEILING_KERNEL = "stream_read_kernel"


def _short(name):
    name = name.split("(")[0]
    for prefix in ("void ", "dq::"):
        if name.startswith(prefix):
            name = name[len(prefix):]
    return name


def _open(path):
    return gzip.open(path, "rt") if path.endswith(".gz") else open(path)


def find(run_dir, suffixes):
    for root, _, files in os.walk(run_dir):
        for f in sorted(files):
            if any(f.endswith(s) for s in suffixes):
                return os.path.join(root, f)
    raise FileNotFoundError(f"no {suffixes} under {run_dir}")


def load_trace(path):
    """[(kernel, start ns, end ns)] in start order."""
    with _open(path) as fh:
        rows = [(_short(r["Kernel_Name"]), int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
                for r in csv.DictReader(fh)]
    rows.sort(key=lambda r: r[1])
    return rows


def load_stats(path):
    with open(path) as fh:
        return {_short(r["Name"]): r for r in csv.DictReader(fh)}


def bench_line(path):
    with open(path) as fh:
        lines = [ln for ln in fh.read().splitlines() if ln.startswith("{")]
    return json.loads(lines[-1])


def timed_legs(rows, protocol):
    """{leg: (timed dispatches, launches per step, steps)} of the timed phase."""
    order, legs = protocol["order"], protocol["legs"]
    per, warm, steps = legs[order[0]]
    n0 = per * (warm + steps)
    starts, run = [], 0
    for i, r in enumerate(rows):
        run = run + 1 if r[0] == CEILING_KERNEL else 0
        if run == n0 and (i + 1 == len(rows) or rows[i + 1][0] != CEILING_KERNEL):
            starts.append(i + 1 - n0)
    if not starts:
        raise ValueError(f"no run of {n0} {CEILING_KERNEL} dispatches opening the timed phase")
    i = starts[-1]
    out = OrderedDict()
    for leg in order:
        per, warm, steps = legs[leg]
        if per is None:  # a leg whose dispatch count the benchmark does not know ends the split
            break
        n = per * (warm + steps)
        seg = rows[i:i + n]
        if len(seg) != n:
            raise ValueError(f"leg {leg}: the trace ends after {len(seg)} of its {n} dispatches")
        out[leg] = (seg[per * warm:], per, steps)
        i += n
    return out


def summarize(rows, line, counter_seq=None):
    legs = timed_legs(rows, line["protocol"])
    byts = {s["leg"]: s["launch_bytes"] for s in counter_seq or []}
    records = []
    for leg, (seg, per, steps) in legs.items():
        span_us = (seg[-1][2] - seg[0][1]) / 1e3
        groups = OrderedDict()
        lb = byts.get(leg)
        if lb is None and leg.endswith(" x5") and leg[:-3] in byts:  # the stack step five times per replay
            lb = byts[leg[:-3]] * 5
        for j, (name, a, b) in enumerate(seg):
            g = groups.setdefault(name, {"d": [], "bytes": 0.0})
            g["d"].append((b - a) / 1e3)
            if lb is not None and len(lb) == per:
                g["bytes"] += lb[j % per]
        for name, g in groups.items():
            d = g["d"]
            rec = {"leg": leg, "kernel": name, "launches_per_step": len(d) // steps, "timed_launches": len(d),
                   "mean_us": statistics.mean(d), "median_us": statistics.median(d), "min_us": min(d),
                   "max_us": max(d), "leg_step_us": span_us / steps}
            if g["bytes"]:
                rec["gbs"] = g["bytes"] / (sum(d) * 1e-6) / 1e9
                rec["bytes_per_launch"] = g["bytes"] / len(d)
            records.append(rec)
    return records


def render(records, line, stats, command, unprofiled=None):
    roof = line.get("roofline", {})
    kern = roof.get("kernel", "")
    out = ["# Engine kernels in the benchmark's timed legs: kernel trace", "",
           "rocprofv3 kernel trace of bench.py with the driver's flags; per timed leg and kernel",
           "instance, the durations of the timed graph replays (warm-up replays dropped). GB/s =",
           "the launches' algorithmic bytes (from the counter pass) / their summed durations.",
           "Leg step us = the leg's timed span / steps under the profiler, which adds per-dispatch",
           "overhead to the legs of many short launches (decode, per-linear): their unprofiled",
           "per-layer times are in the bench line (modes, read_floors), not in that column.",
           "Commands (MI355X, ROCm 7.2):", "", "```"] + command + ["```", ""]
    if kern:
        x5 = [r for r in records if r["leg"] == "C4 stack x5" and r["kernel"].startswith(kern[:-1])]
        st = [v for k, v in stats.items() if k.startswith(kern[:-1])]
        out += [f"Headline kernel `{kern}`:", ""]
        if x5:
            r = x5[0]
            out.append(f"* trace, leg `C4 stack x5` (the launch-duration leg): {r['timed_launches']} timed "
                       f"launches, mean {r['mean_us']:.2f} us, median {r['median_us']:.2f} us")
        out.append(f"* this run's bench line (roofline.mean_launch_us, graph replay time / launches): "
                   f"{roof.get('mean_launch_us', float('nan')):.2f} us; achieved {roof.get('achieved', 0):.0f} GB/s, "
                   f"frac {roof.get('frac', 0):.4f}")
        if unprofiled:
            u = unprofiled["roofline"]
            out.append(f"* the same command without the profiler, same box: mean launch {u['mean_launch_us']:.2f} us, "
                       f"achieved {u['achieved']:.0f} GB/s, frac {u['frac']:.4f}; value {unprofiled['value']:.0f} GB/s")
        if st:
            s = st[0]
            out.append(f"* --stats over the whole run: {s['Calls']} calls, average {float(s['AverageNs']) / 1e3:.2f} us "
                       f"(min {float(s['MinNs']) / 1e3:.2f}, max {float(s['MaxNs']) / 1e3:.2f}): every dispatch of "
                       "the instance, including the eager capture passes, the launch-event pass and the C5 "
                       "stack's launches of other shapes")
        out.append("")
    out += ["| Leg | Kernel | Launches/step | Mean us | Median us | Min | Max | GB/s | % of peak | Leg step us |",
            "|---|---|---|---|---|---|---|---|---|---|"]
    for r in records:
        g = r.get("gbs")
        out.append(f"| {r['leg']} | `{r['kernel']}` | {r['launches_per_step']} | {r['mean_us']:.2f} | "
                   f"{r['median_us']:.2f} | {r['min_us']:.2f} | {r['max_us']:.2f} | "
                   f"{'' if g is None else f'{g:.0f}'} | {'' if g is None else f'{100 * g / PEAK_GBS:.1f}'} | "
                   f"{r['leg_step_us']:.1f} |")
    out.append("")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("run_dir", help="directory holding trace/ (the rocprofv3 output) and bench.json")
    ap.add_argument("--bench", help="bench JSON of the traced run (default <run_dir>/bench.json)")
    ap.add_argument("--counters", help="counter-pass run directory (for bytes per launch)")
    ap.add_argument("--unprofiled", help="bench JSON of the same command run without the profiler, to quote beside")
    ap.add_argument("--out", help="markdown summary to write")
    ap.add_argument("--command", action="append", default=[], help="command line(s) to quote in the summary")
    args = ap.parse_args(argv)
    rows = load_trace(find(args.run_dir, ("kernel_trace.csv", "kernel_trace.csv.gz")))
    stats = load_stats(find(args.run_dir, ("kernel_stats.csv",)))
    line = bench_line(args.bench or os.path.join(args.run_dir, "bench.json"))
    seq = None
    if args.counters:
        with open(os.path.join(args.counters, "FETCH_SIZE.json")) as fh:
            seq = json.loads([ln for ln in fh.read().splitlines() if ln.startswith("{")][-1])["counter_pass"]
    text = render(summarize(rows, line, seq), line, stats, args.command,
                  bench_line(args.unprofiled) if args.unprofiled else None)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text)
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
