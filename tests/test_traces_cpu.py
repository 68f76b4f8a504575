"""dequant_project_amd.traces (host logic): the timed phase found after the
ceiling leg's run of reads, legs split by the recorded protocol, warm-up
replays dropped, bytes per launch from the counter pass."""
import pytest

from dequant_project_amd import traces


def _rows(protocol_legs, order, dur):
    """A trace: build-phase kernels, an earlier (capture) run of the ceiling
    kernel, then the timed legs back to back; kernel k of leg L lasts dur(L, k) us."""
    rows, t = [], 0
    for name in ("randn", "gemv_m1_pipe_kernel<4, false, false, 8>", "stream_read_kernel", "stream_read_kernel",
                 "fill"):
        rows.append((name, t, t + 1000))
        t += 2000
    for leg in order:
        per, warm, steps = protocol_legs[leg]
        for rep in range(warm + steps):
            for k in range(per):
                name = "stream_read_kernel" if leg == "read ceiling" else f"{leg}-k{k % 2}"
                d = dur(leg, k) * (3 if rep < warm else 1)  # warm-up replays are slower: dropped
                rows.append((name, t, t + int(d * 1000)))
                t += int(d * 1000)
    return rows


def test_trace_summary():
    legs = {"read ceiling": [1, 2, 3], "C4 stack": [4, 1, 2], "C4 stack x5": [20, 1, 2]}
    order = ["read ceiling", "C4 stack", "C4 stack x5"]
    rows = _rows(legs, order, lambda leg, k: 10.0 if leg == "read ceiling" else (2.0 if k % 2 == 0 else 4.0))
    line = {"protocol": {"order": order, "legs": legs},
            "roofline": {"kernel": "C4 stack-k0", "mean_launch_us": 2.0, "achieved": 1.0, "frac": 0.1}}
    seq = [{"leg": "C4 stack", "reps": 2, "launch_bytes": [2e6, 4e6, 2e6, 4e6]}]
    recs = traces.summarize(rows, line, seq)
    by = {(r["leg"], r["kernel"]): r for r in recs}
    assert by[("read ceiling", "stream_read_kernel")]["timed_launches"] == 3
    assert by[("read ceiling", "stream_read_kernel")]["mean_us"] == pytest.approx(10.0)
    k0 = by[("C4 stack", "C4 stack-k0")]
    assert (k0["launches_per_step"], k0["timed_launches"], k0["mean_us"]) == (2, 4, pytest.approx(2.0))
    assert k0["gbs"] == pytest.approx(2e6 / 2e-6 / 1e9)  # 2 MB per 2 us launch
    assert by[("C4 stack", "C4 stack-k1")]["gbs"] == pytest.approx(4e6 / 4e-6 / 1e9)
    assert by[("C4 stack x5", "C4 stack x5-k0")]["gbs"] == pytest.approx(1000.0)  # bytes of the stack step x5
    assert by[("C4 stack", "C4 stack-k0")]["leg_step_us"] == pytest.approx(12.0)
    text = traces.render(recs, line, {}, ["cmd"])
    assert "C4 stack x5" in text


def test_trace_summary_needs_the_timed_phase():
    legs = {"read ceiling": [1, 2, 3], "C4 stack": [4, 1, 2]}
    rows = [("stream_read_kernel", i, i + 1) for i in range(4)]  # a run of 4, not the 5 the leg replays
    with pytest.raises(ValueError, match="opening the timed phase"):
        traces.summarize(rows, {"protocol": {"order": ["read ceiling", "C4 stack"], "legs": legs}})
