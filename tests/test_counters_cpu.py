"""dequant_project_amd.counters (host logic): the counter pass's dispatches
split into legs at the delimiter kernels, matched to the launches' bytes by
position, and scaled by the copy calibration."""
import csv
import json
import os

import pytest

from dequant_project_amd import counters

HDR = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _write_run(root, counter, rows, seq):
    d = os.path.join(root, counter, "host", "123")
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "pmc_counter_collection.csv"), "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(HDR)
        for r in rows:
            w.writerow(r)
    with open(os.path.join(root, f"{counter}.json"), "w") as fh:
        fh.write("progress line\n" + json.dumps({"counter_pass": seq}) + "\n")


def _rows(counter, copy_kib, legs):
    """Dispatch rows: a build-phase engine kernel, three copies, then per leg a
    delimiter and its dispatches [(name, kib)] (each split over two rows, as
    the profiler may split a dispatch's counter)."""
    out, did = [], 1
    out.append([did, "void dq::gemv_m1_kernel<4>(dq::KernelBatch)", counter, 5.0])  # before the pass
    did += 1
    for _ in range(3):
        out.append([did, "dq::add_one_kernel(float const*, float*, long)", counter, copy_kib / 2])
        out.append([did, "dq::add_one_kernel(float const*, float*, long)", counter, copy_kib / 2])
        did += 1
    for leg in legs:
        out.append([did, "dq::empty_kernel()", counter, 0.0])
        did += 1
        for name, kib in leg:
            out.append([did, f"void dq::{name}(dq::KernelBatch)", counter, kib * 0.25])
            out.append([did, f"void dq::{name}(dq::KernelBatch)", counter, kib * 0.75])
            did += 1
    return out


def test_counter_summary(tmp_path):
    seq = [{"leg": "read ceiling", "reps": 1, "launch_bytes": [4096.0]},
           {"leg": "C4 stack", "reps": 2, "launch_bytes": [1000.0, 3000.0]}]
    # FETCH: copies read 2^20 KiB at factor 1 -> 1 GiB; report half as many KiB (factor 2)
    fetch_legs = [[("stream_read_kernel", 2.0)],
                  [("pipe<4>", 0.5), ("pipe<4>", 1.5), ("pipe<4>", 0.5), ("pipe<4>", 1.5)]]
    write_legs = [[("stream_read_kernel", 0.0)],
                  [("pipe<4>", 0.01), ("pipe<4>", 0.01), ("pipe<4>", 0.01), ("pipe<4>", 0.01)]]
    _write_run(str(tmp_path), "FETCH_SIZE", _rows("FETCH_SIZE", 2 ** 19, fetch_legs), seq)
    _write_run(str(tmp_path), "WRITE_SIZE", _rows("WRITE_SIZE", 2 ** 20, write_legs), seq)
    records, calib = counters.summarize(str(tmp_path))
    assert calib["fetch_factor"] == pytest.approx(2.0) and calib["write_factor"] == pytest.approx(1.0)
    assert [(r["leg"], r["kernel"], r["launches"]) for r in records] == [
        ("read ceiling", "stream_read_kernel", 1), ("C4 stack", "pipe<4>", 4)]
    ceil, pipe = records
    assert ceil["fetch_bytes_per_launch"] == pytest.approx(4096.0)
    assert ceil["traffic_vs_algorithmic"] == pytest.approx(1.0)
    # launches of 1000 and 3000 algorithmic bytes fetch 1024 and 3072 bytes
    assert pipe["algorithmic_bytes_per_launch"] == pytest.approx(2000.0)
    assert pipe["fetch_bytes_per_launch"] == pytest.approx(2048.0)
    assert pipe["write_bytes_per_launch"] == pytest.approx(10.24)
    assert pipe["traffic_vs_algorithmic"] == pytest.approx((2048.0 + 10.24) / 2000.0)
    text = counters.render(records, calib, ["cmd"])
    rec = json.loads(text.split("```json", 1)[1].split("```", 1)[0])
    assert rec["records"][1]["kernel"] == "pipe<4>"


def test_counter_summary_rejects_mismatched_runs(tmp_path):
    seq = [{"leg": "C4 stack", "reps": 1, "launch_bytes": [1000.0, 3000.0]}]
    _write_run(str(tmp_path), "FETCH_SIZE", _rows("FETCH_SIZE", 2 ** 20, [[("a", 1.0), ("b", 1.0)]]), seq)
    _write_run(str(tmp_path), "WRITE_SIZE", _rows("WRITE_SIZE", 2 ** 20, [[("a", 1.0), ("a", 1.0)]]), seq)
    with pytest.raises(ValueError, match="dispatch 1"):
        counters.summarize(str(tmp_path))
    # a leg with a missing dispatch
    _write_run(str(tmp_path), "WRITE_SIZE", _rows("WRITE_SIZE", 2 ** 20, [[("a", 1.0)]]), seq)
    with pytest.raises(ValueError, match="expected 2"):
        counters.summarize(str(tmp_path))
