"""bench.py (host logic): the warm-up replays of a timed leg. The launch-bound
legs warm up for at least SETTLE_MS of replays estimated at SETTLE_GBS and W
replays at least; the others, the headline's included, for exactly W."""
import math

import bench


def _leg(steps, warmup, step_bytes, settle):
    eager = bench.Leg.eager
    bench.Leg.eager = True  # no graph capture: host logic only
    try:
        return bench.Leg(None, "leg", lambda: None, steps, warmup, step_bytes, settle=settle)
    finally:
        bench.Leg.eager = eager


def test_settle_warmup():
    step = 3_713_007_616  # one C4 step (the decode leg's bytes)
    want = math.ceil(bench.SETTLE_MS * 1e-3 * bench.SETTLE_GBS * 1e9 / step)
    assert want * step / (bench.SETTLE_GBS * 1e9) >= bench.SETTLE_MS * 1e-3
    assert _leg(20, 5, step, True).warmup == want > 5
    assert _leg(20, 5, step, False).warmup == 5          # the headline's legs: exactly W
    assert _leg(20, 500, step, True).warmup == 500       # W when it is the longer
    assert _leg(20, 5, None, True).warmup == 5           # no bytes, no estimate
    assert _leg(20, 5, 25.1e9, True).warmup == 40        # C5's step: 250 ms at 4 TB/s
