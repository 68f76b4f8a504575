#!/usr/bin/env python3
"""Fused dequant-GEMV benchmark on one MI355X.

Workload: the Llama-3-8B decoder linear set --
32 layers x {q 4096->4096, k 4096->1024, v 4096->1024, o 4096->4096,
gate 4096->14336, up 4096->14336, down 14336->4096} -- quantized INT4
asymmetric, group 128, at batch M = 1. Weights are fp16 N(0, 0.02) from a
seeded generator, quantized on the GPU by the engine's packer (3.71 GB packed,
well past the 256 MB Infinity Cache, so every step streams from HBM);
activations are fp16 N(0, 1). Everything is resident in HBM before timing.

One step = one pass of the hot path over the whole stack: all 224 GEMVs, each
with its own synthetic input, captured in one HIP graph. Three launch
structures are timed:

  stack       (headline) the independent GEMVs of the stack as grouped
              launches of up to 16 problems of equal K -- 12 launches of six
              K=4096 projections x 16/6 layers, 2 of 16 down_proj -- i.e. the
              sustained bandwidth of the kernel over the Llama-3-8B layer
              shapes (the reference times independent back-to-back GEMV calls
              the same way, scripts/bench_dequant_kernel.py:119-168);
  decode      what a decoder launches given a Llama layer's data
              dependencies: q|k|v grouped (same input), o, gate|up grouped,
              down -- 4 launches per layer, 128 per step;
  per_linear  the QuantLinear drop-in path: one launch per projection.

Measurement protocol (why the timed replays see the steady state):
  * Every input of the timed legs is built and every graph captured before
    any timing starts, and nothing is freed until the end. Freeing device
    memory (torch.cuda.empty_cache) lets the driver clear the freed VRAM in
    the background, which costs the next ~10 ms per freed GB about 3% of the
    bandwidth; graph capture and host-side building leave the GPU idle, after
    which the power management takes ~20 ms of load to bring the memory path
    back to its steady clocks (the first replays then run up to 15% slower).
  * The timed legs then run back to back on one stream with no host
    synchronization between them. The first leg is the streaming-read
    ceiling (a measurement of its own, reported below, long enough to cover
    that ramp); the headline stack follows immediately with its W warm-up
    and K timed replays.
  * The launch-bound legs (C4 decode and per_linear, their read floors, the
    prologue legs, C5 decode) warm up for at least SETTLE_MS of estimated
    replay time (their bytes at 4 TB/s), W replays at least: right after the
    headline's stack leg the same decode graph ran 7% slower (32.9 against
    30.7 us/layer, its kernels within 1%: the gaps between launches grow),
    and reached its steady figure after a few hundred ms of launches. The
    warm-up replays of every leg are in protocol.legs.
  * roofline.achieved is the dominant kernel's own duration: a leg replays
    the stack step five times per graph (70 launches back to back, so the
    per-replay launch overhead is spread thin), and replay time / launches is
    the mean launch duration, the figure rocprofv3's kernel trace reports
    for graph-replayed kernels (dequant_project_amd/traces.py summarizes that
    trace per leg). The launch-event hook (hipExtLaunchKernelGGL start/stop
    events around each eager launch) is reported beside it.

Printed: ONE JSON line on stdout (progress goes to stderr).
  value            stack-mode algorithmic bytes per step / step time, GB/s
                   (the byte_model accounting: packed weights + scales +
                   zeros + x + y)
  roofline         the headline's kernel: algorithmic bytes per launch / its
                   mean kernel duration; traffic: HBM bytes per launch from the
                   committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary of the
                   counter pass (a static figure, not measured in this run)
  ceilings         measured streaming-read ceiling and empty-kernel gap
  read_floors      per launch structure (stack, decode, per_linear): the same
                   launches as plain streaming reads of their bytes, i.e. what
                   the structure would take at the read rate with its launch
                   overheads (and the GEMV's time over it)
  cpu_baseline     the reference's CPU torch path (oracle/cpu_path.py) on the
                   host cores: C4 one layer (value), rows for C1-C5, 1 thread
  other_format_stacks / batch_stacks  the same stack step in INT8 and INT2,
                   and the INT4 stack at M = 2, 4, 8 (C4's other batch sizes)
  gemm_small_stacks  the fused small GEMM over the stack at M = 16, 64, with
                   the reference's dequantize + F.linear timed beside it
  decode_with_fused_prologues  the decode launches with RMSNorm / SwiGLU
                   fused in, against the same launches without
  c5_llama3_70b_stack  BASELINE.json's C5 (~25 GB), stack and decode
  single_configs   C1, C2 (M = 1, 4), C3, each in a graph of distinct copies
  format_axis      the reference's microbenchmark table on the C4 shapes: per
                   shape and format, per-call time in a graph of distinct
                   copies, with fp16 F.linear and the speed-up over it
                   (scripts/bench_dequant_kernel.py:61-78, 119-168)

  python bench.py [--gpus 1] [--steps 20] [--warmup 5]
  python bench.py --counters --calibrate-copy --no-cpu-baseline --steps 2
      the counter pass for rocprofv3 --pmc runs (no graphs, no timing;
      dequant_project_amd/counters.py turns two such runs into the traffic
      summary)
"""

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fused dequant-GEMV HBM GB/s (% of MI355X peak) + µs/layer, INT2/4/8, batch 1"
PEAK_GBS = 8000.0
LAYERS = 32
HIDDEN, KV, INTER = 4096, 1024, 14336
PROJS = [("q_proj", HIDDEN, HIDDEN), ("k_proj", KV, HIDDEN), ("v_proj", KV, HIDDEN),
         ("o_proj", HIDDEN, HIDDEN), ("gate_proj", INTER, HIDDEN), ("up_proj", INTER, HIDDEN),
         ("down_proj", HIDDEN, INTER)]
GROUPS = [("qkv", ("q_proj", "k_proj", "v_proj")), ("o", ("o_proj",)),
          ("gate_up", ("gate_proj", "up_proj")), ("down", ("down_proj",))]
MALL_BYTES = 256 * 2 ** 20
CEILING_BYTES = 4 * 2 ** 30      # streaming-read ceiling buffer
CEILING_WARM, CEILING_REPS = 20, 40
EMPTY_LAUNCHES = 1000
LAUNCH_LEG_STEPS = 5             # stack steps per replay of the launch-duration leg
SETTLE_MS = 250                  # minimum warm-up of the launch-bound legs (see the protocol above)
SETTLE_GBS = 4000.0              # the rate that warm-up is estimated at
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "dq_kernels_bench_legs_traffic.md")

# a Llama-3-70B-shape stack in mixed precision
C5_LAYERS = 80
C5_HIDDEN, C5_KV, C5_INTER, C5_VOCAB = 8192, 1024, 28672, 128256


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def summarize(samples):
    s = sorted(samples)
    n = len(s)
    return {"median": statistics.median(s), "p25": s[n // 4], "p75": s[(3 * n) // 4],
            "min": s[0], "max": s[-1], "n": n}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=LAYERS, help=argparse.SUPPRESS)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true",
                    help="time the C4 INT4 modes only (no other formats, batches, C5, single configs, format axis)")
    ap.add_argument("--modes", default="stack,decode,per_linear",
                    help="comma-separated step structures to time (stack is the headline)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 1 GiB device copy, the engine's add_one kernel (rocprof FETCH_SIZE / "
                         "WRITE_SIZE calibration)")
    ap.add_argument("--counters", action="store_true",
                    help="counter pass for rocprofv3 --pmc runs: every leg's step run eagerly STEPS times (no "
                         "graphs, no timing), an empty kernel before each leg as a delimiter; prints the "
                         "algorithmic bytes of every launch in order")
    return ap.parse_args()


class Engine:
    """The engine's entry points used here: the torch extension for launches,
    the C ABI for the launch plan (kernel instance names), the launch-event
    hook and the measurement kernels."""

    def __init__(self, torch):
        from dequant_project_amd import _native

        self.torch = torch
        self.ext = _native.ext()
        self.capi = _native.capi()
        self.native = _native

    def gemv_group(self, xs, pws):
        cfg = pws[0].config
        if len(pws) == 1:
            pw = pws[0]
            return [self.ext.gemv(xs[0], pw.qweight, pw.scales, pw.zeros, cfg.bits,
                                  cfg.effective_group_size(pw.shape[1]), cfg.symmetric,
                                  cfg.layout == "interleaved")]
        return self.ext.gemv_batched(xs, [p.qweight for p in pws], [p.scales for p in pws],
                                     [p.zeros for p in pws], cfg.bits,
                                     [p.config.effective_group_size(p.shape[1]) for p in pws], cfg.symmetric,
                                     cfg.layout == "interleaved")

    def kernel_name(self, xs, pws):
        """Kernel instance a launch of these problems uses (dq_gemv_plan)."""
        n = len(pws)
        arr = (self.native.DqGemvProblem * n)()
        for i, (x, p) in enumerate(zip(xs, pws)):
            arr[i].N, arr[i].K = p.shape
            arr[i].group_size = p.config.effective_group_size(p.shape[1])
        wk, rows, kind = (ctypes.c_int * n)(), ctypes.c_int(), ctypes.c_int()
        cfg = pws[0].config
        m = xs[0].shape[0]
        st = self.capi.dq_gemv_plan(arr, n, m, cfg.bits, wk, ctypes.byref(rows), ctypes.byref(kind))
        self.native.check(st)
        fmt = f"{cfg.bits}, {str(cfg.symmetric).lower()}, {str(cfg.layout == 'interleaved').lower()}"
        if kind.value == 1:
            return f"gemv_quad_kernel<{fmt}, {rows.value // 4}, {1 if m <= 4 else 2}>", tuple(wk)
        if kind.value == 7:
            return f"gemv_mx_pipe_kernel<{fmt}, {rows.value}, 2>", tuple(wk)
        if kind.value == 4:
            return f"gemv_m1_pipe_kernel<{fmt}, {rows.value}>", tuple(wk)
        if kind.value == 8:
            return f"gemv_m1_pipe_split_kernel<{fmt}, {rows.value}, {wk[0]}>", tuple(wk)
        if kind.value == 6:
            return f"gemv_m1_kernel<{fmt}, {rows.value}, false> (kept x)", tuple(wk)
        return f"gemv_m1_kernel<{fmt}, {rows.value}, {'true' if kind.value == 3 else 'false'}>", tuple(wk)

    def stream(self):
        return self.torch.cuda.current_stream().cuda_stream

    def stream_read(self, buf, sink):
        self.native.check(self.capi.dq_stream_read(buf.data_ptr(), buf.numel() * buf.element_size(),
                                                   sink.data_ptr(), self.stream()))

    def empty_kernel(self):
        self.native.check(self.capi.dq_empty_kernel(self.stream()))

    def add_one(self, src, dst):
        self.native.check(self.capi.dq_add_one(src.data_ptr(), dst.data_ptr(), src.numel(), self.stream()))


# ----------------------------------------------------------------- building
def quantize_random(torch, gen, n, k, cfg):
    from dequant_project_amd.packer import quantize_tensor

    w = torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02
    pw = quantize_tensor(w, cfg)
    del w
    return pw


def build_stack(torch, layers, seed=20251201, cfg=None):
    from dequant_project_amd.packer import QuantConfig

    cfg = cfg or QuantConfig(4, 128, False, "sequential")
    gen = torch.Generator(device="cuda").manual_seed(seed)
    stack = [{name: quantize_random(torch, gen, n, k, cfg) for name, n, k in PROJS} for _ in range(layers)]
    return cfg, stack, make_xs(torch, layers, 1, gen)


def make_xs(torch, layers, m, gen):
    """Per layer, the fp16 N(0, 1) inputs [m, K] of its four launch roles."""
    return [{"qkv": torch.randn(m, HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
             "o": torch.randn(m, HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
             "gate_up": torch.randn(m, HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
             "down": torch.randn(m, INTER, generator=gen, device="cuda", dtype=torch.float16)}
            for _ in range(layers)]


def step_launches(stack, xs, mode):
    """[(role, [x...], [pw...])] of one step."""
    out = []
    if mode == "stack":
        by_k = {}
        for layer, x in zip(stack, xs):
            for role, names in GROUPS:
                for n in names:
                    by_k.setdefault(layer[n].shape[1], []).append((x[role], layer[n]))
        for k, items in by_k.items():
            for i in range(0, len(items), 16):
                chunk = items[i:i + 16]
                out.append((f"K={k}", [c[0] for c in chunk], [c[1] for c in chunk]))
        return out
    for layer, x in zip(stack, xs):
        for role, names in GROUPS:
            if mode == "decode":
                out.append((role, [x[role]] * len(names), [layer[n] for n in names]))
            else:
                for n in names:
                    out.append((role, [x[role]], [layer[n]]))
    return out


def launch_bytes(xs, pws):
    from dequant_project_amd import byte_model as bm

    total = 0
    for x, p in zip(xs, pws):
        c = p.config
        total += bm.gemv_call_bytes(p.shape[0], p.shape[1], c.bits, c.group_size, c.symmetric, x.shape[0])
    return total


def kernel_instances(eng, launches):
    """Kernel instance of every launch of a step (dq_gemv_plan) -> {name: [bytes...]}."""
    inst = {}
    for _, x, p in launches:
        name, _ = eng.kernel_name(x, p)
        inst.setdefault(name, []).append(launch_bytes(x, p))
    return inst


def capture(torch, fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


# ------------------------------------------------------------------ timing
class Leg:
    """One timed leg: the step function `fn` captured in a graph, replayed
    `warmup` times, then `steps` times between events. Replays are only
    enqueued here; `result` reads the events after the single synchronization
    that ends the timed phase. `launch_bytes`: the algorithmic bytes of each
    kernel launch of one step, in launch order (the counter pass maps them to
    the profiler's dispatches). With Leg.eager set (the counter pass) nothing
    is captured: the pass calls `fn` directly."""

    eager = False

    def __init__(self, torch, name, fn, steps, warmup, step_bytes=None, meta=None, layers=None, launch_bytes=None,
                 settle=False):
        self.torch, self.name, self.fn = torch, name, fn
        self.graph = None if Leg.eager else capture(torch, fn)
        if settle and step_bytes:  # at least SETTLE_MS of replays at the estimated rate
            warmup = max(warmup, math.ceil(SETTLE_MS * 1e-3 * SETTLE_GBS * 1e9 / step_bytes))
        self.steps, self.warmup = steps, warmup
        self.step_bytes, self.meta, self.layers = step_bytes, meta or {}, layers
        self.launch_bytes = launch_bytes
        self.evs = None

    def enqueue(self):
        for _ in range(self.warmup):
            self.graph.replay()
        self.evs = [self.torch.cuda.Event(enable_timing=True) for _ in range(self.steps + 1)]
        self.evs[0].record()
        for i in range(self.steps):
            self.graph.replay()
            self.evs[i + 1].record()

    def result(self):
        per = [self.evs[i].elapsed_time(self.evs[i + 1]) for i in range(self.steps)]
        ms = self.evs[0].elapsed_time(self.evs[-1]) / self.steps
        out = {"ms_per_step": ms, "step_ms": summarize(per)}
        if self.step_bytes:
            out.update(bytes_per_step=self.step_bytes, gbs=self.step_bytes / (ms * 1e-3) / 1e9,
                       pct_peak=100 * self.step_bytes / (ms * 1e-3) / 1e9 / PEAK_GBS)
        if self.layers:
            out["us_per_layer"] = ms * 1e3 / self.layers
        out.update(self.meta)
        return out


def gemv_leg(torch, eng, name, launches, steps, warmup, layers, settle=False):
    step_bytes = sum(launch_bytes(x, p) for _, x, p in launches)

    def fn():
        for _, x, p in launches:
            eng.gemv_group(x, p)

    meta = {"launches_per_step": len(launches),
            "kernel_instances": {k: len(v) for k, v in kernel_instances(eng, launches).items()}}
    return Leg(torch, name, fn, steps, warmup, step_bytes, meta, layers, [launch_bytes(x, p) for _, x, p in launches],
               settle=settle)


def read_floor_leg(torch, eng, name, flat, sink, sizes, steps, warmup, layers, settle=False):
    """A plain streaming read (stream_read_kernel) of each launch's
    algorithmic bytes, in the same launch structure: consecutive regions of
    `flat` (wrapping at its end), one read launch per GEMV launch."""
    views, off = [], 0
    for s in sizes:
        n = (int(s) + 15) // 16 * 16
        if off + n > flat.numel():
            off = 0
        views.append(flat[off:off + n])
        off += n

    def fn():
        for v in views:
            eng.stream_read(v, sink)

    return Leg(torch, name, fn, steps, warmup, sum(v.numel() for v in views), layers=layers,
               launch_bytes=[v.numel() for v in views], settle=settle)


def kernel_durations(torch, eng, launches, reps):
    """Per-launch kernel durations (us) of `launches`, run eagerly `reps` times
    on the current stream, each launch timed by the engine's launch-event hook
    (hipExtLaunchKernelGGL start/stop events bracket the kernel itself). The
    launches go straight through the C ABI (dq_gemv_batched) with problem
    arrays and outputs prepared beforehand, so the host issues a launch in a
    few microseconds and the GPU runs them back to back, as in the graph (the
    torch entry points allocate their outputs per call, and a host slower than
    the kernels would leave the GPU idle between them)."""
    lib, nat = eng.capi, eng.native
    prepared = []
    for _, xs, pws in launches:
        arr = (nat.DqGemvProblem * len(pws))()
        ys = []
        for i, (x, p) in enumerate(zip(xs, pws)):
            y = torch.empty(x.shape[0], p.shape[0], dtype=torch.float16, device="cuda")
            ys.append(y)
            arr[i].x, arr[i].qweight, arr[i].scales = x.data_ptr(), p.qweight.data_ptr(), p.scales.data_ptr()
            arr[i].zeros = None if p.zeros is None else p.zeros.data_ptr()
            arr[i].y = y.data_ptr()
            arr[i].N, arr[i].K = p.shape
            arr[i].group_size = p.config.effective_group_size(p.shape[1])
        c = pws[0].config
        prepared.append((arr, len(pws), xs[0].shape[0], c.bits, int(c.symmetric), int(c.layout == "interleaved"), ys))
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in launches]
    for a, b in evs:  # an event's handle exists once it has been recorded
        a.record()
        b.record()
    stream = eng.stream()
    out = []
    for _ in range(reps + 1):  # the first pass warms the launch path and is dropped
        for (a, b), (arr, n, m, bits, sym, inter, _) in zip(evs, prepared):
            nat.check(lib.dq_set_launch_events(a.cuda_event, b.cuda_event))
            nat.check(lib.dq_gemv_batched(arr, n, m, bits, sym, inter, stream))
        torch.cuda.synchronize()
        out.append([a.elapsed_time(b) * 1e3 for a, b in evs])
    return out[1:]


def profiled_traffic(kernel, leg="C4 stack"):
    """HBM bytes per launch of `kernel` in `leg` from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of the counter pass (copy-calibrated,
    dequant_project_amd/counters.py), or None if it holds no such record."""
    try:
        text = open(TRAFFIC_PROFILE).read()
        recs = json.loads(text.split("```json", 1)[1].split("```", 1)[0])["records"]
    except (OSError, IndexError, ValueError, KeyError):
        return None, None
    for rec in recs:  # the engine names instances without the trailing default template arguments
        if rec["leg"] == leg and (rec["kernel"] == kernel or rec["kernel"].startswith(kernel[:-1] + ",")):
            return rec["traffic_bytes_per_launch"], rec
    return None, None


# ------------------------------------------------------------ extra legs
def c5_build(torch):
    """80 layers of q/k/v/o in INT4 g128 asym and gate/up/down in INT2 g64
    asym, plus an INT8 per-channel sym lm_head 8192 -> 128256 (~25 GB
    packed), from seeded fp16 N(0, 0.02) weights quantized on the GPU one
    tensor at a time; x fp16 N(0, 1), batch 1."""
    from dequant_project_amd.packer import QuantConfig

    attn, mlp, head = QuantConfig(4, 128, False), QuantConfig(2, 64, False), QuantConfig(8, None, True)
    gen = torch.Generator(device="cuda").manual_seed(20251206)
    shapes = {"q_proj": (C5_HIDDEN, C5_HIDDEN, attn), "k_proj": (C5_KV, C5_HIDDEN, attn),
              "v_proj": (C5_KV, C5_HIDDEN, attn), "o_proj": (C5_HIDDEN, C5_HIDDEN, attn),
              "gate_proj": (C5_INTER, C5_HIDDEN, mlp), "up_proj": (C5_INTER, C5_HIDDEN, mlp),
              "down_proj": (C5_HIDDEN, C5_INTER, mlp)}
    stack = [{name: quantize_random(torch, gen, n, k, c) for name, (n, k, c) in shapes.items()}
             for _ in range(C5_LAYERS)]
    lm_head = quantize_random(torch, gen, C5_VOCAB, C5_HIDDEN, head)
    xs = [{"qkv": torch.randn(1, C5_HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
           "o": torch.randn(1, C5_HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
           "gate_up": torch.randn(1, C5_HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
           "down": torch.randn(1, C5_INTER, generator=gen, device="cuda", dtype=torch.float16)} for _ in stack]
    x_head = torch.randn(1, C5_HIDDEN, generator=gen, device="cuda", dtype=torch.float16)
    return stack, lm_head, xs, x_head


def c5_launches(stack, lm_head, xs, x_head):
    """Grouped launches of equal format and K ("stack") and the decoder's
    launches ("decode": q|k|v, o, gate|up, down per layer), then the lm_head."""
    groups = {}
    for layer, x in zip(stack, xs):
        for role, names in GROUPS:
            for n in names:
                p = layer[n]
                groups.setdefault((p.config.bits, p.shape[1]), []).append((x[role], p))
    out = {"stack": [("g", [c[0] for c in items[i:i + 16]], [c[1] for c in items[i:i + 16]])
                     for items in groups.values() for i in range(0, len(items), 16)],
           "decode": [(role, [x[role]] * len(names), [layer[n] for n in names])
                      for layer, x in zip(stack, xs) for role, names in GROUPS]}
    for mode in out:
        out[mode].append(("lm_head", [x_head], [lm_head]))
    return out


# name, N, K, (bits, group_size, symmetric), M
SINGLE_CONFIGS = [("C1", 4096, 4096, (4, 128, False), 1), ("C2", 11008, 4096, (8, None, True), 1),
                  ("C2_M4", 11008, 4096, (8, None, True), 4), ("C3", 4096, 11008, (2, 64, False), 1)]


def single_copies(torch, n, k, cfg, seed, outliers=False):
    """The reference's rotating-copy working set (>= 8 x the 256 MB Infinity
    Cache in place of its L2, and at least one copy per layer,
    scripts/bench_dequant_kernel.py:119-126): one seeded weight quantized,
    then cloned into distinct device copies (the timing depends on the
    memory, not on the values)."""
    from dequant_project_amd.packer import PackedWeight, quantize_tensor

    gen = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02
    if outliers:  # C3: 0.1% of the entries at +-10 sigma
        cnt = max(1, (n * k) // 1000)
        idx = torch.randint(0, n * k, (cnt,), generator=gen, device="cuda")
        sign = torch.where(torch.rand(cnt, generator=gen, device="cuda") < 0.5, -1.0, 1.0)
        w.view(-1)[idx] = (sign * 0.2).to(torch.float16)
    first = quantize_tensor(w, cfg)
    del w
    copies = max(LAYERS, math.ceil(8 * MALL_BYTES / first.nbytes))
    return [first] + [PackedWeight(first.qweight.clone(), first.scales.clone(),
                                   None if first.zeros is None else first.zeros.clone(), first.config, first.shape)
                      for _ in range(copies - 1)]


GEMM_MS = (16, 32, 64)  # batch rows of the small-GEMM legs


def gemm_dispatch_bytes(x, p):
    """Algorithmic bytes of each kernel launch of one gemm_small call, in
    launch order: one launch, or, for a call the engine splits along K
    (dq_gemm_small_plan), the walk (weights, scales, zeros, activations) and
    the launch that sums its partial tiles (the output; the partials it reads
    are traffic beyond the algorithmic bytes)."""
    from dequant_project_amd import _native

    lib = _native.capi()
    pr = _native.DqGemvProblem()
    pr.N, pr.K = p.shape
    pr.group_size = p.config.effective_group_size(p.shape[1])
    splits = (ctypes.c_int * 1)()
    _native.check(lib.dq_gemm_small_plan(ctypes.byref(pr), 1, x.shape[0], p.config.bits, splits))
    total = launch_bytes([x], [p])
    if splits[0] == 1:
        return [total]
    out = x.shape[0] * p.shape[0] * 2
    return [total - out, out]


def gemm_stack_leg(torch, stack, m, steps, warmup):
    """The fused small GEMM (quant_linear.gemm_small) over every projection of
    the stack at m rows (a prefill chunk through all layers) as one leg, and
    its items (x, weight)."""
    from dequant_project_amd.quant_linear import gemm_small

    gen = torch.Generator(device="cuda").manual_seed(20251204 + m)
    xs = {k: torch.randn(m, k, generator=gen, device="cuda", dtype=torch.float16) for k in (HIDDEN, INTER)}
    items = [(xs[p.shape[1]], p) for layer in stack for _, p in sorted(layer.items())]
    per_launch = [b for x, p in items for b in gemm_dispatch_bytes(x, p)]

    def fused():
        for x, p in items:
            gemm_small(x, p)

    return Leg(torch, f"gemm M={m}", fused, steps, warmup, sum(per_launch), layers=len(stack),
               launch_bytes=per_launch), items


def gemm_stack(torch, stack, m, steps, warmup):
    """gemm_stack_leg timed in one graph, against the reference's M > 8 path
    (dequantize + F.linear) timed eagerly with HIP events (each of its GEMMs
    is tens of microseconds)."""
    import torch.nn.functional as F

    from dequant_project_amd.quant_linear import dequantize_cuda

    leg, items = gemm_stack_leg(torch, stack, m, steps, warmup)
    leg.enqueue()

    def reference():
        for x, p in items:
            F.linear(x, dequantize_cuda(p))

    reference()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ref = []
    for _ in range(max(3, steps // 4)):
        a.record()
        reference()
        b.record()
        torch.cuda.synchronize()
        ref.append(a.elapsed_time(b))
    r = leg.result()
    ref_ms = statistics.median(ref)
    r.update(M=m, dequantize_plus_linear_ms_per_step=ref_ms, speedup_vs_dequantize_plus_linear=ref_ms / r["ms_per_step"])
    return r


# label, (bits, group_size, symmetric, layout) or None for fp16 F.linear
FORMAT_AXIS = [("fp16 F.linear", None), ("INT8 g128 sym", (8, 128, True, "sequential")),
               ("INT4 g128 sym", (4, 128, True, "sequential")), ("INT4 g128 asym", (4, 128, False, "sequential")),
               ("INT4 g32 sym", (4, 32, True, "sequential")), ("INT4 per-chan sym", (4, None, True, "sequential")),
               ("INT4 g128 sym inter", (4, 128, True, "interleaved"))]
FORMAT_SHAPES = [("q/o_proj", HIDDEN, HIDDEN), ("k/v_proj", KV, HIDDEN), ("gate/up_proj", INTER, HIDDEN),
                 ("down_proj", HIDDEN, INTER)]


def format_axis_legs(torch, eng, steps, warmup):
    """The legs of format_axis: one per (shape, format)."""
    import torch.nn.functional as F

    from dequant_project_amd import byte_model as bm
    from dequant_project_amd.packer import PackedWeight, QuantConfig, quantize_tensor

    gen = torch.Generator(device="cuda").manual_seed(20251207)
    pairs = []
    for label, n, k in FORMAT_SHAPES:
        w = torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02
        x = torch.randn(1, k, generator=gen, device="cuda", dtype=torch.float16)
        for fmt, spec in FORMAT_AXIS:
            if spec is None:
                copies = max(LAYERS, math.ceil(8 * MALL_BYTES / (n * k * 2)))
                ws = [w.clone() for _ in range(copies)]

                def fn(ws=ws, x=x):
                    for wi in ws:
                        F.linear(x, wi)
                call_bytes = n * k * 2 + k * 2 + n * 2
                kernel = "torch F.linear (fp16)"
            else:
                cfg = QuantConfig(*spec)
                first = quantize_tensor(w, cfg)
                copies = max(LAYERS, math.ceil(8 * MALL_BYTES / first.nbytes))
                ws = [first] + [PackedWeight(first.qweight.clone(), first.scales.clone(),
                                             None if first.zeros is None else first.zeros.clone(), cfg, first.shape)
                                for _ in range(copies - 1)]

                def fn(ws=ws, x=x):
                    for p in ws:
                        eng.gemv_group([x], [p])
                call_bytes = bm.gemv_call_bytes(n, k, cfg.bits, cfg.group_size, cfg.symmetric, 1)
                kernel = eng.kernel_name([x], [first])[0]
            leg = Leg(torch, f"{label} {fmt}", fn, steps, warmup, launch_bytes=None if spec is None else
                      [call_bytes] * copies)
            pairs.append((label, n, k, fmt, copies, call_bytes, kernel, leg, ws))
    return pairs


def format_axis(torch, eng, steps, warmup):
    """The reference's microbenchmark (scripts/bench_dequant_kernel.py:61-78,
    119-168) on the Llama-3-8B projection shapes: per (shape, format) a graph
    of n_copies = max(32, ceil(8 x 256 MB / bytes)) back-to-back calls over
    distinct copies, M = 1; per-call time = replay time / n_copies (median,
    p25, p75 over the timed replays); fp16 F.linear over the fp16 weight is
    the row every speed-up is measured against. Every pair is built and
    captured first, then all are timed back to back."""
    pairs = format_axis_legs(torch, eng, steps, warmup)
    torch.cuda.synchronize()
    for p in pairs:
        p[7].enqueue()
    torch.cuda.synchronize()
    rows, base = [], {}
    for label, n, k, fmt, copies, call_bytes, kernel, leg, _ in pairs:
        r = leg.result()
        us = r["step_ms"]["median"] * 1e3 / copies
        base.setdefault(label, us)
        rows.append({"shape": label, "format": fmt, "N": n, "K": k, "copies": copies, "bytes_per_call": call_bytes,
                     "us_median": us, "us_p25": r["step_ms"]["p25"] * 1e3 / copies,
                     "us_p75": r["step_ms"]["p75"] * 1e3 / copies, "gbs": call_bytes / (us * 1e-6) / 1e9,
                     "pct_peak": 100 * call_bytes / (us * 1e-6) / 1e9 / PEAK_GBS,
                     "floor_us": call_bytes / (PEAK_GBS * 1e9) * 1e6, "speedup_vs_fp16": base[label] / us,
                     "kernel": kernel})
    return rows


# ------------------------------------------------------------ counter pass
def counter_pass(torch, args, eng, stack, ceiling, legs):
    """The kernels of every leg, run eagerly for rocprofv3 counter collection
    (--pmc FETCH_SIZE / WRITE_SIZE with a kernel filter on the engine's
    kernels): per leg an empty kernel (the delimiter the summary splits
    dispatches on), then the leg's step `args.steps` times. The ceiling read
    runs once (a read of known size: a second calibration beside the copy).
    Prints {"counter_pass": [{leg, reps, launch_bytes}, ...]}: the algorithmic
    bytes of each launch of one step, in dispatch order."""
    seq = []

    def run(name, leg, reps):
        eng.empty_kernel()
        for _ in range(reps):
            leg.fn()
        torch.cuda.synchronize()
        seq.append({"leg": name, "reps": reps, "launch_bytes": leg.launch_bytes})
        log(f"counter pass: {name} x{reps}")

    run("read ceiling", ceiling, 1)
    for name, leg in legs.items():
        if name != "C4 stack x5":  # the stack step again
            run(name, leg, args.steps)
    if not args.no_extra:
        for m in GEMM_MS:
            leg, _ = gemm_stack_leg(torch, stack, m, args.steps, args.warmup)
            run(f"gemm M={m}", leg, args.steps)
        for label, n, k, fmt, copies, call_bytes, kernel, leg, _ in format_axis_legs(torch, eng, args.steps,
                                                                                       args.warmup):
            if leg.launch_bytes is not None:  # fp16 F.linear runs no engine kernel
                run(f"axis {label} {fmt}", leg, 1)
    print(json.dumps({"counter_pass": seq}), flush=True)
    return 0


# ------------------------------------------------------------ CPU baseline
def cpu_baseline(torch, c4_layer, singles, c5_layer, budget_s=30.0):
    """The reference's CPU torch path (oracle/cpu_path.py: unpack -> dequantize
    -> fp32 F.linear), timed with time.perf_counter on this host's cores
    (torch.get_num_threads()): 3 warm-ups, then the
    median and p25/p75 of up to 20 repetitions (fewer for rows whose single
    repetition would overrun the time budget; the count is recorded),
    'dequant + matmul' and 'matmul only' (the fp32 weight materialized
    beforehand). C4 and C5 time one layer (7 linears; the C5 row excludes the
    lm_head) and scale by the layer count; a 1-thread row repeats C1.
    value = the C4 layer's GB/s."""
    from oracle import cpu_path

    def host(p):
        return (p.qweight.cpu(), p.scales.cpu(), None if p.zeros is None else p.zeros.cpu(), p.config, p.shape)

    def row(name, items, m, layers, reps_cap, warm):
        gen = torch.Generator().manual_seed(3)
        ws = [host(p) for p in items]
        xs = [torch.randn(m, shape[1], generator=gen, dtype=torch.float16) for *_, shape in ws]
        nbytes = sum(launch_bytes([x], [p]) for x, p in zip(xs, items))

        def deq_mm():
            for x, (qw, sc, ze, c, shape) in zip(xs, ws):
                cpu_path.gemv(x, qw, sc, ze, c.bits, c.effective_group_size(shape[1]), c.symmetric,
                              c.layout == "interleaved")

        t0 = time.perf_counter()
        deq_mm()
        one = time.perf_counter() - t0
        for _ in range(warm - 1):
            deq_mm()
        reps = int(max(3, min(reps_cap, budget_s / 8 / max(one, 1e-4))))
        samples = []
        for _ in range(reps):
            t0 = time.perf_counter()
            deq_mm()
            samples.append(time.perf_counter() - t0)
        wf = [cpu_path.dequantize(qw, sc, ze, c.bits, c.effective_group_size(shape[1]), c.symmetric,
                                  c.layout == "interleaved", shape[1]).float() for qw, sc, ze, c, shape in ws]
        mm = []
        for _ in range(reps):
            t0 = time.perf_counter()
            for x, w in zip(xs, wf):
                torch.nn.functional.linear(x.float(), w)
            mm.append(time.perf_counter() - t0)
        st, sm = summarize(samples), summarize(mm)
        return {"config": name, "M": m, "threads": torch.get_num_threads(), "warmups": warm, "reps": reps,
                "layers_scaled": layers, "bytes": nbytes,
                "us_median": st["median"] * 1e6, "us_p25": st["p25"] * 1e6, "us_p75": st["p75"] * 1e6,
                "matmul_only_us_median": sm["median"] * 1e6, "gbs": nbytes / st["median"] / 1e9,
                "s_per_step_scaled": st["median"] * layers if layers else None}

    threads = torch.get_num_threads()
    rows = [row("C1", [singles["C1"]], 1, None, 20, 3), row("C2", [singles["C2"]], 1, None, 20, 3),
            row("C2", [singles["C2"]], 4, None, 20, 3), row("C3", [singles["C3"]], 1, None, 20, 3),
            row("C4 (one layer of 32)", [c4_layer[n] for n, _, _ in PROJS], 1, LAYERS, 20, 3),
            row("C5 (one layer of 80, lm_head excluded)", list(c5_layer.values()), 1, C5_LAYERS, 3, 1)]
    torch.set_num_threads(1)
    try:
        rows.append(row("C1", [singles["C1"]], 1, None, 10, 3))
    finally:
        torch.set_num_threads(threads)
    c4 = rows[4]
    return {"value": c4["gbs"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": (f"one Llama-3-8B layer (7 linears, {c4['bytes'] / 1e6:.1f} MB packed INT4 g128 asym, M=1) "
                       f"of the benchmark stack, unpack -> dequantize -> fp32 F.linear (oracle/cpu_path.py), "
                       f"median of {c4['reps']} after 3 warm-ups; rows for C1-C5 and a 1-thread C1 row"),
            "us_per_layer": c4["us_median"], "matmul_only_us_per_layer": c4["matmul_only_us_median"],
            "os_cpu_count": os.cpu_count(), "rows": rows}


# ------------------------------------------------------------------- main
def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    import torch

    from dequant_project_amd.packer import QuantConfig

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    eng = Engine(torch)
    Leg.eager = args.counters
    torch.backends.cuda.matmul.allow_tf32 = False
    log(f"device: {torch.cuda.get_device_name(0)}  torch {torch.__version__}")
    extra = not args.no_extra

    if args.calibrate_copy:
        # a plain copy of known size for the counters: the engine's add_one
        # kernel over 2^28 floats reads 1 GiB and writes 1 GiB
        src = torch.ones(2 ** 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            eng.add_one(src, dst)
        torch.cuda.synchronize()
        log("calibration copy: 1 GiB read + 1 GiB write, 3 times")
        del src, dst

    # ---- 1. build every input of the timed legs (resident until the end)
    t0 = time.perf_counter()
    cfg, stack, xs = build_stack(torch, args.layers)
    ceiling_buf = torch.empty(CEILING_BYTES // 4, dtype=torch.int32, device="cuda").random_()
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    if extra:
        other = {key: build_stack(torch, args.layers, seed=20251202, cfg=c)
                 for key, c in (("INT8 per-channel sym", QuantConfig(8, None, True)),
                                ("INT2 g64 asym", QuantConfig(2, 64, False)))}
        bgen = torch.Generator(device="cuda").manual_seed(20251203)
        batch_xs = {m: make_xs(torch, args.layers, m, bgen) for m in (2, 4, 8)}
        pgen = torch.Generator(device="cuda").manual_seed(20251205)
        gamma = torch.rand(HIDDEN, generator=pgen, device="cuda", dtype=torch.float16) + 0.5
        ups = [torch.randn(1, INTER, generator=pgen, device="cuda", dtype=torch.float16) for _ in stack]
        c5 = c5_build(torch)
        singles = {name: single_copies(torch, n, k, QuantConfig(*spec), seed=n * 7 + k, outliers=name == "C3")
                   for name, n, k, spec, _ in SINGLE_CONFIGS if name != "C2_M4"}
        sgen = torch.Generator(device="cuda").manual_seed(20251208)
        single_x = {name: torch.randn(m, k, generator=sgen, device="cuda", dtype=torch.float16)
                    for name, n, k, _, m in SINGLE_CONFIGS}
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    log(f"built every input in {build_s:.1f}s")

    # ---- 2. capture every graph (host only)
    modes = [m.strip() for m in args.modes.split(",") if m.strip()]
    if "stack" not in modes:
        modes.insert(0, "stack")
    c4_launches = {mode: step_launches(stack, xs, mode) for mode in modes}
    legs = {f"C4 {mode}": gemv_leg(torch, eng, mode, c4_launches[mode], args.steps, args.warmup, args.layers,
                                   settle=mode != "stack")
            for mode in modes}
    # the floor of each structure: a plain read of every launch's bytes
    flat = ceiling_buf.view(torch.uint8)
    for mode in modes:
        legs[f"read floor {mode}"] = read_floor_leg(torch, eng, f"read floor {mode}", flat, sink,
                                                    legs[f"C4 {mode}"].launch_bytes, args.steps, args.warmup,
                                                    args.layers, settle=mode != "stack")
    # the headline's launch-duration leg: the same step five times in one
    # graph, so the per-replay launch overhead is spread over 70 launches
    legs["C4 stack x5"] = gemv_leg(torch, eng, "stack x5", c4_launches["stack"] * LAUNCH_LEG_STEPS, args.steps,
                                   args.warmup, args.layers * LAUNCH_LEG_STEPS)
    singles_meta = {}
    if extra:
        from dequant_project_amd import fused

        for key, (_, ostack, oxs) in other.items():
            legs[f"stack {key}"] = gemv_leg(torch, eng, key, step_launches(ostack, oxs, "stack"), args.steps,
                                            args.warmup, args.layers)
        for m, mxs in batch_xs.items():
            legs[f"stack M={m}"] = gemv_leg(torch, eng, f"M={m}", step_launches(stack, mxs, "stack"), args.steps,
                                            args.warmup, args.layers)
        legs["prologue plain"] = gemv_leg(torch, eng, "plain", step_launches(stack, xs, "decode"), args.steps,
                                          args.warmup, args.layers, settle=True)

        def run_fused():
            for li, (layer, x) in enumerate(zip(stack, xs)):
                fused.gemv_rmsnorm(x["qkv"], gamma, 1e-5, [layer["q_proj"], layer["k_proj"], layer["v_proj"]])
                eng.gemv_group([x["o"]], [layer["o_proj"]])
                fused.gemv_rmsnorm(x["gate_up"], gamma, 1e-5, [layer["gate_proj"], layer["up_proj"]])
                fused.gemv_swiglu(x["down"], ups[li], layer["down_proj"])

        # the fused launches read gamma (q|k|v, gate|up) or up (down) besides
        # the plain launches' bytes
        extra = [3 * HIDDEN * 2, 0, 2 * HIDDEN * 2, INTER * 2]
        legs["prologue fused"] = Leg(torch, "fused", run_fused, args.steps, args.warmup,
                                     legs["prologue plain"].step_bytes, layers=args.layers,
                                     launch_bytes=[b + extra[i % 4] for i, b in
                                                   enumerate(legs["prologue plain"].launch_bytes)], settle=True)

        def rmsnorm(x):  # transformers' LlamaRMSNorm in torch ops
            h = x.float()
            h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-5)
            return gamma * h.to(torch.float16)

        def run_unfused():
            for li, (layer, x) in enumerate(zip(stack, xs)):
                h = rmsnorm(x["qkv"])
                eng.gemv_group([h] * 3, [layer["q_proj"], layer["k_proj"], layer["v_proj"]])
                eng.gemv_group([x["o"]], [layer["o_proj"]])
                h = rmsnorm(x["gate_up"])
                eng.gemv_group([h] * 2, [layer["gate_proj"], layer["up_proj"]])
                eng.gemv_group([torch.nn.functional.silu(x["down"]) * ups[li]], [layer["down_proj"]])

        # what a decoder runs without the fused prologues: the same launches
        # plus the RMSNorm and SwiGLU as torch ops (not counted in its bytes;
        # the leg is timed last, as its kernel count per step is torch's)
        unfused = Leg(torch, "unfused", run_unfused, args.steps, args.warmup, legs["prologue plain"].step_bytes,
                      layers=args.layers, launch_bytes=legs["prologue plain"].launch_bytes, settle=True)
        for mode, ls in c5_launches(*c5).items():
            legs[f"C5 {mode}"] = gemv_leg(torch, eng, mode, ls, args.steps, args.warmup, C5_LAYERS,
                                          settle=mode == "decode")
        for name, n, k, spec, m in SINGLE_CONFIGS:
            pws = singles["C2" if name == "C2_M4" else name]
            x = single_x[name]

            def fn(pws=pws, x=x):
                for p in pws:
                    eng.gemv_group([x], [p])

            legs[f"single {name}"] = Leg(torch, name, fn, 10, 2,
                                         launch_bytes=[launch_bytes([x], [pws[0]])] * len(pws))
            singles_meta[name] = (n, k, spec, m, len(pws), launch_bytes([x], [pws[0]]),
                                  eng.kernel_name([x], [pws[0]])[0])
        legs["prologue unfused"] = unfused

    def ceiling_fn():
        eng.stream_read(ceiling_buf, sink)

    ceiling = Leg(torch, "read ceiling", ceiling_fn, CEILING_REPS, CEILING_WARM, ceiling_buf.numel() * 4,
                  launch_bytes=[ceiling_buf.numel() * 4])

    def empty_fn():
        for _ in range(EMPTY_LAUNCHES):
            eng.empty_kernel()

    empty = Leg(torch, "empty kernels", empty_fn, 10, 3, launch_bytes=[0] * EMPTY_LAUNCHES)
    torch.cuda.synchronize()
    if args.counters:
        return counter_pass(torch, args, eng, stack, ceiling, legs)
    log(f"captured {len(legs) + 2} graphs")

    # ---- 3. timed legs, back to back, one synchronization at the end
    ceiling.enqueue()
    for leg in legs.values():
        leg.enqueue()
    empty.enqueue()
    torch.cuda.synchronize()

    results = {key: leg.result() for key, leg in legs.items()}
    ceil_r = ceiling.result()
    ceil_gbs = ceiling.step_bytes / (ceil_r["step_ms"]["median"] * 1e-3) / 1e9
    empty_r = empty.result()
    ceilings = {"stream_read_gbs": ceil_gbs, "stream_read_pct_peak": 100 * ceil_gbs / PEAK_GBS,
                "stream_read_bytes": ceiling.step_bytes, "stream_read_reps": CEILING_REPS,
                "stream_read_step_ms": ceil_r["step_ms"],
                "stream_read_kernel": "stream_read_kernel (dq_stream_read: non-temporal, 1 KiB per wave and load)",
                "empty_kernel_us_per_launch": empty_r["step_ms"]["median"] * 1e3 / EMPTY_LAUNCHES,
                "empty_kernel_launches_per_graph": EMPTY_LAUNCHES}
    log(f"read ceiling {ceil_gbs:.0f} GB/s ({100 * ceil_gbs / PEAK_GBS:.1f}%), empty kernel "
        f"{ceilings['empty_kernel_us_per_launch']:.2f} us per launch in a graph")
    read_floors = {}
    for mode in modes:
        r = results[f"C4 {mode}"]
        f = results.pop(f"read floor {mode}")
        read_floors[mode] = {"ms_per_step": f["ms_per_step"], "us_per_layer": f["us_per_layer"], "gbs": f["gbs"],
                             "pct_peak": f["pct_peak"], "gemv_time_vs_floor": r["ms_per_step"] / f["ms_per_step"]}
        log(f"mode {mode}: {r['ms_per_step']:.3f} ms/step  {r['gbs']:.1f} GB/s  {r['us_per_layer']:.2f} us/layer  "
            f"({r['launches_per_step']} launches); a plain read of the same launches {f['us_per_layer']:.2f} "
            f"us/layer ({f['gbs']:.0f} GB/s)")

    # ---- 4. the headline kernel's launch duration
    # (a) live, over timed replays: the launch-duration leg replays the stack
    #     step LAUNCH_LEG_STEPS times per graph; its launches run back to back,
    #     so replay time / launches is the mean launch duration (what
    #     rocprofv3's kernel trace reports for graph-replayed kernels)
    # (b) the launch-event hook on eager launches, for reference: it brackets
    #     each kernel with start/stop markers, whose own cost is included
    launches = c4_launches["stack"]
    names = [eng.kernel_name(x, p)[0] for _, x, p in launches]
    per_name = {}
    for i, nm in enumerate(names):
        per_name.setdefault(nm, []).append(i)
    dominant = max(per_name, key=lambda nm: sum(launch_bytes(launches[i][1], launches[i][2]) for i in per_name[nm]))
    dom_idx = per_name[dominant]
    dom_bytes = sum(launch_bytes(launches[i][1], launches[i][2]) for i in dom_idx) / len(dom_idx)
    x5 = results.pop("C4 stack x5")
    graph_launch_us = x5["ms_per_step"] * 1e3 / (LAUNCH_LEG_STEPS * len(launches))
    durs = kernel_durations(torch, eng, launches, args.steps)
    hook_us = statistics.mean(d[i] for d in durs for i in dom_idx)
    single_instance = len(per_name) == 1
    dom_us = graph_launch_us if single_instance else hook_us
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    traffic, trec = profiled_traffic(dominant)
    roofline = {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBS, "unit": "GB/s", "frac": achieved / PEAK_GBS,
                "traffic": traffic, "kernel": dominant, "bytes_per_launch": dom_bytes, "mean_launch_us": dom_us,
                "launches_per_step": len(dom_idx),
                "method": ((f"algorithmic bytes per launch / mean launch duration in timed graph replays of "
                            f"{LAUNCH_LEG_STEPS} consecutive stack steps ({args.steps} replays after {args.warmup} "
                            "warm-up, HIP events on the launch stream); the step runs one kernel instance")
                           if single_instance else
                           f"algorithmic bytes per launch / mean kernel duration over {args.steps} eager passes, "
                           "each launch bracketed by hipExtLaunchKernelGGL start/stop events (dq_set_launch_events)"),
                "graph_launch_us": graph_launch_us, "eager_hook_launch_us": hook_us,
                "step_launch_interval_us": results["C4 stack"]["ms_per_step"] * 1e3 / len(launches),
                "traffic_unit": "bytes per launch",
                "traffic_source": ("static: rocprofv3 FETCH_SIZE + WRITE_SIZE of this kernel on this workload, "
                                   "copy-calibrated, profiles/" + os.path.basename(TRAFFIC_PROFILE)
                                   if traffic else "no committed counter summary for this kernel")}
    if trec:
        roofline["traffic_vs_algorithmic"] = traffic / trec["algorithmic_bytes_per_launch"]
    log(f"dominant kernel {dominant}: {len(dom_idx)} launches/step, {dom_bytes / 1e6:.1f} MB/launch, "
        f"{dom_us:.2f} us/launch, {achieved:.1f} GB/s ({100 * achieved / PEAK_GBS:.1f}%); eager hook "
        f"{hook_us:.2f} us/launch")

    other_stacks, batch_stacks, prologue, c5_r, single_r = {}, {}, None, None, {}
    if extra:
        for key in other:
            r = other_stacks[key] = results[f"stack {key}"]
            log(f"stack {key}: {r['ms_per_step']:.3f} ms/step  {r['gbs']:.1f} GB/s  {r['us_per_layer']:.2f} us/layer")
        for m in batch_xs:
            r = batch_stacks[f"M={m}"] = results[f"stack M={m}"]
            log(f"stack INT4 M={m}: {r['ms_per_step']:.3f} ms/step  {r['gbs']:.1f} GB/s  "
                f"{r['us_per_layer']:.2f} us/layer")
        prologue = {"plain": results["prologue plain"], "fused_prologues": results["prologue fused"],
                    "unfused_prologues": results["prologue unfused"],
                    "bytes_per_step": legs["prologue plain"].step_bytes,
                    "note": "plain: the decode launches alone (activations prepared); fused_prologues: RMSNorm "
                            "(q|k|v, gate|up) and SwiGLU (down) inside the launches; unfused_prologues: the plain "
                            "launches plus RMSNorm and SwiGLU as torch ops, what a decoder runs without the fusion"}
        log(f"decode launches: plain {prologue['plain']['us_per_layer']:.2f} us/layer, with fused prologues "
            f"{prologue['fused_prologues']['us_per_layer']:.2f} us/layer, with the prologues as torch ops "
            f"{prologue['unfused_prologues']['us_per_layer']:.2f} us/layer")
        c5_r = {"layers": C5_LAYERS, "stack": results["C5 stack"], "decode": results["C5 decode"]}
        log(f"C5: stack {c5_r['stack']['ms_per_step']:.3f} ms/step {c5_r['stack']['gbs']:.1f} GB/s "
            f"{c5_r['stack']['us_per_layer']:.2f} us/layer; decode {c5_r['decode']['ms_per_step']:.3f} ms/step "
            f"{c5_r['decode']['gbs']:.1f} GB/s")
        for name, (n, k, spec, m, copies, b, kern) in singles_meta.items():
            st = results[f"single {name}"]["step_ms"]
            us = st["median"] * 1e3 / copies
            single_r[name] = {"shape": [n, k], "M": m, "format": f"INT{spec[0]} g{spec[1] or 'pc'} "
                              f"{'sym' if spec[2] else 'asym'}", "copies": copies, "bytes_per_call": b,
                              "us_per_call": us, "us_p25": st["p25"] * 1e3 / copies, "us_p75": st["p75"] * 1e3 / copies,
                              "gbs": b / (us * 1e-6) / 1e9, "pct_peak": 100 * b / (us * 1e-6) / 1e9 / PEAK_GBS,
                              "kernel": kern}
            log(f"{name}: {us:.2f} us/call ({single_r[name]['gbs']:.0f} GB/s) in a graph of {copies} copies")

    # ---- 5. legs that build and time in place (their builds reuse cached memory)
    gemm, axis = {}, []
    if extra:
        for m in GEMM_MS:
            g = gemm[f"M={m}"] = gemm_stack(torch, stack, m, args.steps, args.warmup)
            log(f"gemm_small stack M={m}: {g['ms_per_step']:.3f} ms/step  {g['gbs']:.1f} GB/s  "
                f"(dequantize + F.linear {g['dequantize_plus_linear_ms_per_step']:.3f} ms/step, "
                f"{g['speedup_vs_dequantize_plus_linear']:.2f}x)")
        axis = format_axis(torch, eng, args.steps, args.warmup)
        for r in axis:
            log(f"  {r['shape']:<13}{r['format']:<21}{r['us_median']:8.2f} us {r['gbs']:8.0f} GB/s "
                f"{r['pct_peak']:5.1f}%  {r['speedup_vs_fp16']:5.2f}x vs fp16")

    # ---- 6. CPU baseline (needs the extra legs' single-config weights)
    cpu = None
    if extra and not args.no_cpu_baseline:
        t0 = time.perf_counter()
        cpu = cpu_baseline(torch, stack[0], {k: singles[k][0] for k in ("C1", "C2", "C3")}, c5[0][0])
        log(f"cpu baseline: {cpu['value']:.3f} GB/s on {cpu['cores']} threads ({time.perf_counter() - t0:.1f}s)")

    head_r = results["C4 stack"]
    gbs = head_r["gbs"]
    line = {
        "metric": METRIC, "value": gbs, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head_r["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int4 codes -> fp16 (q-z), fp16 x fp16 products, fp32 accumulate",
        "data": "synthetic (seeded fp16 N(0,0.02) weights quantized on the GPU; fp16 N(0,1) activations)",
        "config": {"workload": "C4: Llama-3-8B decoder linear set (32 layers x q,k,v,o,gate,up,down), "
                               "INT4 g128 asym, M=1",
                   "layers": args.layers, "batch": 1, "bytes_per_step": head_r["bytes_per_step"],
                   "launches_per_step": head_r["launches_per_step"],
                   "grouping": "stack: launches of up to 16 independent GEMVs of equal K"},
        "pct_of_peak": 100 * gbs / PEAK_GBS,
        "us_per_layer": head_r["us_per_layer"],
        "roofline": roofline,
        "cpu_baseline": cpu,
        "ceilings": ceilings,
        "protocol": {"build_s": build_s, "order": ["read ceiling"] + list(legs) + ["empty kernels"],
                     "legs": {name: [None if name == "prologue unfused" else len(leg.launch_bytes), leg.warmup,
                                     leg.steps] for name, leg in
                              [("read ceiling", ceiling)] + list(legs.items()) + [("empty kernels", empty)]},
                     "note": "every input built and every graph captured before timing; nothing freed; the legs "
                             "replayed back to back with one synchronization at the end"},
        "modes": {mode: results[f"C4 {mode}"] for mode in modes},
        "read_floors": read_floors,
        "other_format_stacks": other_stacks,
        "batch_stacks": batch_stacks,
        "gemm_small_stacks": gemm,
        "decode_with_fused_prologues": prologue,
        "c5_llama3_70b_stack": c5_r,
        "single_configs": single_r,
        "format_axis": axis,
    }
    print(json.dumps(line, default=lambda o: sorted(o) if isinstance(o, set) else str(o)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
