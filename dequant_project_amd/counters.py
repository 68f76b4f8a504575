"""HBM traffic of every engine kernel the benchmark runs, from two rocprofv3
counter runs of bench.py's counter pass (one FETCH_SIZE, one WRITE_SIZE),
each calibrated against a plain device copy of known size.

    rocprofv3 --pmc FETCH_SIZE --kernel-include-regex "dq::" --output-format csv \\
        -d <run>/FETCH_SIZE -o pmc -- \\
        python3 bench.py --counters --calibrate-copy --no-cpu-baseline --steps 2 > <run>/FETCH_SIZE.json
    (the same with WRITE_SIZE)
    python3 -m dequant_project_amd.counters <run> [--out profiles/<name>.md]

The counter pass (bench.py --counters) runs each leg's step eagerly after an
empty kernel, and prints the algorithmic bytes of every launch of one step in
dispatch order; the empty kernels split the profiler's dispatches into legs,
and the bytes are matched to the dispatches by position. The calibration copy
(the engine's add_one kernel over 2^28 floats: 1 GiB read and 1 GiB
written, three times, before any leg) gives the factor from each counter's
KiB to bytes; the ceiling read (stream_read_kernel over 4 GiB) is reported
as a check of the FETCH factor. Only the engine's kernels are counted, not
the thousands of torch kernels and runtime copies that build the inputs (two
runs that also counted the runtime's copy kernels ended in a crash inside
the profiler).

Traffic per launch = FETCH_SIZE x fetch factor + WRITE_SIZE x write factor;
the ratio to the algorithmic bytes (the byte_model accounting: packed
weights, scales, zeros, activations, outputs) shows re-read or wasted bytes
(1.00: every byte fetched once).
"""
import argparse
import csv
import glob
import json
import os
import sys
from collections import OrderedDict

COPY_BYTES = 2 ** 30
DELIMITER = "empty_kernel"
CALIBRATION = "add_one_kernel"


def _short(name):
    name = name.split("(")[0]
    for prefix in ("void ", "dq::"):
        if name.startswith(prefix):
            name = name[len(prefix):]
    return name


def load_dispatches(run_dir, counter):
    """[(dispatch id, kernel name, KiB)] of one counter run, in dispatch order
    (values of one dispatch summed over the rows the profiler splits it into)."""
    files = glob.glob(os.path.join(run_dir, counter, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise FileNotFoundError(f"no counter_collection.csv under {os.path.join(run_dir, counter)}")
    per = OrderedDict()
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                if r["Counter_Name"] != counter:
                    continue
                key = int(r["Dispatch_Id"])
                if key not in per:
                    per[key] = [r["Kernel_Name"], 0.0]
                per[key][1] += float(r["Counter_Value"])
    return [(k, v[0], v[1]) for k, v in sorted(per.items())]


def load_sequence(run_dir, counter):
    path = os.path.join(run_dir, f"{counter}.json")
    with open(path) as fh:
        lines = [ln for ln in fh.read().splitlines() if ln.startswith("{")]
    return json.loads(lines[-1])["counter_pass"]


def split_legs(dispatches, seq):
    """Engine dispatches per leg: the last len(seq) delimiters open the legs."""
    engine = dispatches  # the profiler's kernel filter keeps the engine's kernels only
    marks = [i for i, d in enumerate(engine) if _short(d[1]) == DELIMITER]
    if len(marks) < len(seq):
        raise ValueError(f"{len(marks)} delimiter kernels for {len(seq)} legs")
    marks = marks[-len(seq):]
    out = []
    for j, leg in enumerate(seq):
        end = marks[j + 1] if j + 1 < len(seq) else len(engine)
        body = engine[marks[j] + 1:end]
        expect = leg["reps"] * len(leg["launch_bytes"])
        if len(body) != expect:
            raise ValueError(f"leg {leg['leg']}: {len(body)} dispatches, expected {expect}")
        out.append(body)
    return out


def calibration(dispatches):
    kib = [d[2] for d in dispatches if _short(d[1]) == CALIBRATION]
    if not kib:
        raise ValueError("no calibration copy in the run (bench.py --calibrate-copy)")
    mean = sum(kib) / len(kib)
    return COPY_BYTES / (mean * 1024.0), mean, len(kib)


def summarize(run_dir):
    fetch = load_dispatches(run_dir, "FETCH_SIZE")
    write = load_dispatches(run_dir, "WRITE_SIZE")
    seq = load_sequence(run_dir, "FETCH_SIZE")
    if [s["launch_bytes"] for s in seq] != [s["launch_bytes"] for s in load_sequence(run_dir, "WRITE_SIZE")]:
        raise ValueError("the two counter runs ran different launch sequences")
    ff, fcp, fn = calibration(fetch)
    wf, wcp, wn = calibration(write)
    legs_f, legs_w = split_legs(fetch, seq), split_legs(write, seq)
    records = []
    for leg, bf, bw in zip(seq, legs_f, legs_w):
        L = len(leg["launch_bytes"])
        groups = OrderedDict()
        for i, (df, dw) in enumerate(zip(bf, bw)):
            name = _short(df[1])
            if name != _short(dw[1]):
                raise ValueError(f"leg {leg['leg']}: dispatch {i} is {name} in one run, {_short(dw[1])} in the other")
            g = groups.setdefault(name, {"n": 0, "alg": 0.0, "fetch": 0.0, "write": 0.0})
            g["n"] += 1
            g["alg"] += leg["launch_bytes"][i % L]
            g["fetch"] += df[2] * 1024.0 * ff
            g["write"] += dw[2] * 1024.0 * wf
        for name, g in groups.items():
            records.append({"leg": leg["leg"], "kernel": name, "launches": g["n"],
                            "algorithmic_bytes_per_launch": g["alg"] / g["n"],
                            "fetch_bytes_per_launch": g["fetch"] / g["n"],
                            "write_bytes_per_launch": g["write"] / g["n"],
                            "traffic_bytes_per_launch": (g["fetch"] + g["write"]) / g["n"],
                            "traffic_vs_algorithmic": (g["fetch"] + g["write"]) / g["alg"]})
    calib = {"fetch_factor": ff, "fetch_copy_kib": fcp, "fetch_copies": fn,
             "write_factor": wf, "write_copy_kib": wcp, "write_copies": wn}
    return records, calib


def render(records, calib, command):
    lines = ["# Engine kernels over the benchmark's legs: HBM traffic (FETCH_SIZE, WRITE_SIZE)", "",
             "Every kernel instance the benchmark runs, per leg, from two rocprofv3 counter runs of",
             "bench.py's counter pass (eager launches of each leg's step; one counter per run),",
             "calibrated against a plain copy of known size (the engine's add_one kernel over 2^28",
             "floats: 1 GiB read, 1 GiB written). Commands (MI355X, ROCm 7.2):", "", "```"] + command + ["```", "",
             "| Counter | copy kernel (KiB/dispatch, n) | bytes it moved | factor |", "|---|---|---|---|",
             f"| FETCH_SIZE | {calib['fetch_copy_kib']:.1f} ({calib['fetch_copies']}) | 1 GiB read | "
             f"{calib['fetch_factor']:.4f} |",
             f"| WRITE_SIZE | {calib['write_copy_kib']:.1f} ({calib['write_copies']}) | 1 GiB written | "
             f"{calib['write_factor']:.4f} |", "",
             "Traffic = FETCH x factor + WRITE x factor, per launch (mean over the leg's launches of",
             "that kernel); algorithmic = the byte_model accounting of the same launches.", "",
             "| Leg | Kernel | Launches | Algorithmic MB/launch | Fetch MB | Write MB | Traffic / algorithmic |",
             "|---|---|---|---|---|---|---|"]
    for r in records:
        lines.append(f"| {r['leg']} | `{r['kernel']}` | {r['launches']} | {r['algorithmic_bytes_per_launch'] / 1e6:.3f} "
                     f"| {r['fetch_bytes_per_launch'] / 1e6:.3f} | {r['write_bytes_per_launch'] / 1e6:.4f} "
                     f"| {r['traffic_vs_algorithmic']:.3f} |")
    slim = [{"leg": r["leg"], "kernel": r["kernel"], "launches": r["launches"],
             "algorithmic_bytes_per_launch": round(r["algorithmic_bytes_per_launch"]),
             "traffic_bytes_per_launch": round(r["traffic_bytes_per_launch"])} for r in records]
    cal = {k: round(v, 4) if isinstance(v, float) else v for k, v in calib.items()}
    lines += ["", "```json", json.dumps({"calibration": cal, "records": slim}), "```", ""]
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("run_dir", help="directory holding FETCH_SIZE/, WRITE_SIZE/ and FETCH_SIZE.json, WRITE_SIZE.json")
    ap.add_argument("--out", help="markdown summary to write")
    ap.add_argument("--command", action="append", default=[], help="command line(s) to quote in the summary")
    args = ap.parse_args(argv)
    records, calib = summarize(args.run_dir)
    text = render(records, calib, args.command)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text)
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
