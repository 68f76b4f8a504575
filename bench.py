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
              shapes, with launch overhead amortized (the reference times
              independent back-to-back GEMV calls the same way,
              scripts/bench_dequant_kernel.py:119-168);
  decode      what a decoder launches given a Llama layer's data
              dependencies: q|k|v grouped (same input), o, gate|up grouped,
              down -- 4 launches per layer, 128 per step;
  per_linear  the QuantLinear drop-in path: one launch per projection.

Printed: ONE JSON line on stdout (progress goes to stderr).
  value       stack-mode algorithmic bytes per step / step time, GB/s (the
              byte_model accounting: packed weights + scales + zeros + x + y)
  roofline    the dominant kernel instance of the stack step: algorithmic
              bytes per launch / its mean launch duration, the latter from HIP
              events around the timed graph replays divided by the launches
              (the stack step runs one kernel instance), against 8 TB/s
  cpu_baseline  the reference's CPU torch path (oracle/cpu_path.py) on one
              layer of the same stack, on this host's cores
  other_format_stacks / batch_stacks  the same stack step in INT8 and INT2,
              and the INT4 stack at M = 2, 4, 8 (C4's other batch sizes)
  gemm_small_stacks  the fused small GEMM over the stack at M = 16, 64, with
              the reference's dequantize + F.linear timed beside it
  decode_with_fused_prologues  the decode launches with RMSNorm / SwiGLU
              fused in, against the same launches without
  c5_llama3_70b_stack  BASELINE.json's C5: the Llama-3-70B shapes, INT4
              attention, INT2 MLP, INT8 lm_head (~25 GB), stack and decode
              launch structures

  python bench.py [--gpus 1] [--steps 20] [--warmup 100]
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
    # ~70 ms of replays: the GPU needs ~45 ms of this load after the stack is
    # built before the step time settles (the first replays run ~15% slower)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--layers", type=int, default=LAYERS, help=argparse.SUPPRESS)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the C1/C2/C3 single-config runs")
    ap.add_argument("--modes", default="stack,decode,per_linear",
                    help="comma-separated step structures to time (stack is the headline)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 1 GiB device copy (rocprof FETCH_SIZE/WRITE_SIZE calibration)")
    return ap.parse_args()


class Engine:
    """The engine's entry points used here: the torch extension for launches
    and the C ABI's launch plan (to name the kernel instance of a launch)."""

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
        return f"gemv_m1_kernel<{fmt}, {rows.value}, {'true' if kind.value == 3 else 'false'}>", tuple(wk)


def build_stack(torch, layers, seed=20251201, cfg=None):
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    cfg = cfg or QuantConfig(4, 128, False, "sequential")
    gen = torch.Generator(device="cuda").manual_seed(seed)
    stack = []
    for _ in range(layers):
        layer = {}
        for name, n, k in PROJS:
            w = torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02
            layer[name] = quantize_tensor(w, cfg)
            del w
        stack.append(layer)
    return cfg, stack, make_xs(torch, layers, 1, gen)


def make_xs(torch, layers, m, gen):
    """Per layer, the fp16 N(0, 1) inputs [m, K] of its four launch roles."""
    xs = []
    for _ in range(layers):
        xs.append({"qkv": torch.randn(m, HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
                   "o": torch.randn(m, HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
                   "gate_up": torch.randn(m, HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
                   "down": torch.randn(m, INTER, generator=gen, device="cuda", dtype=torch.float16)})
    return xs


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


def time_graph(torch, graph, steps, warmup):
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    evs[0].record()
    for i in range(steps):
        graph.replay()
        evs[i + 1].record()
    torch.cuda.synchronize()
    per = [evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]
    return evs[0].elapsed_time(evs[-1]) / steps, per


def run_mode(torch, eng, stack, xs, mode, steps, warmup):
    launches = step_launches(stack, xs, mode)
    step_bytes = sum(launch_bytes(x, p) for _, x, p in launches)

    def fn():
        for _, x, p in launches:
            eng.gemv_group(x, p)

    graph = capture(torch, fn)
    ms, per = time_graph(torch, graph, steps, warmup)
    del graph
    return launches, step_bytes, ms, per


def kernel_instances(eng, launches):
    """Kernel instance of every launch of a step (dq_gemv_plan) -> {name: [bytes...]}."""
    inst = {}
    for _, x, p in launches:
        name, _ = eng.kernel_name(x, p)
        inst.setdefault(name, []).append(launch_bytes(x, p))
    return inst


def cpu_baseline(torch, stack):
    """The reference's CPU torch path (unpack -> dequantize -> fp32 F.linear) on layer 0."""
    from oracle import cpu_path

    layer = stack[0]
    cpu = {n: (p.qweight.cpu(), p.scales.cpu(), p.zeros.cpu(), p.config, p.shape) for n, p in layer.items()}
    gen = torch.Generator().manual_seed(3)
    xs = {n: torch.randn(1, shape[1], generator=gen, dtype=torch.float16) for n, (*_, shape) in cpu.items()}
    layer_bytes = sum(launch_bytes([xs[n]], [p]) for n, p in layer.items())

    def one_layer(matmul_only=None):
        for n, (qw, sc, ze, c, shape) in cpu.items():
            if matmul_only is None:
                cpu_path.gemv(xs[n], qw, sc, ze, c.bits, c.effective_group_size(shape[1]), c.symmetric,
                              c.layout == "interleaved")
            else:
                torch.nn.functional.linear(xs[n].float(), matmul_only[n])

    threads = torch.get_num_threads()
    t0 = time.perf_counter()
    one_layer()  # warm-up
    warm = time.perf_counter() - t0
    reps = max(3, min(20, int(15.0 / max(warm, 1e-3))))
    samples = []
    for _ in range(reps):
        t0 = time.perf_counter()
        one_layer()
        samples.append(time.perf_counter() - t0)
    med = statistics.median(samples)
    weights = {n: cpu_path.dequantize(qw, sc, ze, c.bits, c.effective_group_size(shape[1]), c.symmetric,
                                      c.layout == "interleaved", shape[1]).float()
               for n, (qw, sc, ze, c, shape) in cpu.items()}
    mm = []
    for _ in range(reps):
        t0 = time.perf_counter()
        one_layer(weights)
        mm.append(time.perf_counter() - t0)
    return {"value": layer_bytes / med / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": (f"one Llama-3-8B layer (7 linears, {layer_bytes / 1e6:.1f} MB packed INT4 g128 asym, M=1) "
                       f"of the benchmark stack, unpack -> dequantize -> fp32 F.linear "
                       f"(oracle/cpu_path.py), median of {reps} after 1 warm-up"),
            "us_per_layer": med * 1e6, "matmul_only_us_per_layer": statistics.median(mm) * 1e6,
            "os_cpu_count": os.cpu_count()}


def single_config(torch, eng, name, n, k, cfg, m, reps=10):
    """The reference's rotating-copy microbenchmark for one shape (working set
    >= 8 x the 256 MB Infinity Cache): per-call graph time and kernel time."""
    from dequant_project_amd.packer import quantize_tensor

    gen = torch.Generator(device="cuda").manual_seed(n * 7 + k)
    first = quantize_tensor(torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02, cfg)
    copies = max(4, math.ceil(8 * MALL_BYTES / first.nbytes))
    pws = [first] + [quantize_tensor(torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02,
                                     cfg) for _ in range(copies - 1)]
    x = torch.randn(m, k, generator=gen, device="cuda", dtype=torch.float16)

    def fn():
        for p in pws:
            eng.gemv_group([x], [p])

    graph = capture(torch, fn)
    ms, per = time_graph(torch, graph, reps, 2)
    b = launch_bytes([x], [first])
    us = statistics.median(per) * 1e3 / copies
    res = {"shape": [n, k], "M": m, "format": f"INT{cfg.bits} g{cfg.group_size or 'pc'} "
           f"{'sym' if cfg.symmetric else 'asym'}", "copies": copies, "bytes_per_call": b,
           "us_per_call": us, "gbs": b / (us * 1e-6) / 1e9, "pct_peak": 100 * b / (us * 1e-6) / 1e9 / PEAK_GBS,
           "kernel": eng.kernel_name([x], [first])[0]}
    del graph, pws, first
    torch.cuda.empty_cache()
    return name, res


def gemm_stack(torch, stack, m, steps, warmup):
    """The fused small GEMM (quant_linear.gemm_small) over every projection of
    the stack at m rows (a prefill chunk through all layers), in one graph,
    against the reference's M > 8 path (dequantize + F.linear) timed eagerly
    with HIP events (each of its GEMMs is tens of microseconds)."""
    import torch.nn.functional as F

    from dequant_project_amd.quant_linear import dequantize_cuda, gemm_small

    gen = torch.Generator(device="cuda").manual_seed(20251204 + m)
    xs = {k: torch.randn(m, k, generator=gen, device="cuda", dtype=torch.float16) for k in (HIDDEN, INTER)}
    items = [(xs[p.shape[1]], p) for layer in stack for _, p in sorted(layer.items())]
    step_bytes = sum(launch_bytes([x], [p]) for x, p in items)

    def fused():
        for x, p in items:
            gemm_small(x, p)

    graph = capture(torch, fused)
    ms, per = time_graph(torch, graph, steps, warmup)
    del graph

    def reference():
        for x, p in items:
            F.linear(x, dequantize_cuda(p))

    reference()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ref = []
    for _ in range(max(3, steps // 4)):
        a.record()
        reference()
        b.record()
        torch.cuda.synchronize()
        ref.append(a.elapsed_time(b))
    ref_ms = statistics.median(ref)
    return {"M": m, "bytes_per_step": step_bytes, "ms_per_step": ms, "step_ms": summarize(per),
            "gbs": step_bytes / (ms * 1e-3) / 1e9, "pct_peak": 100 * step_bytes / (ms * 1e-3) / 1e9 / PEAK_GBS,
            "us_per_layer": ms * 1e3 / len(stack),
            "dequantize_plus_linear_ms_per_step": ref_ms, "speedup_vs_dequantize_plus_linear": ref_ms / ms}


def prologue_decode(torch, eng, stack, xs, steps, warmup):
    """The decode launch structure (q|k|v, o, gate|up, down per layer) with the
    RMSNorm prologue fused into q|k|v and gate|up and the SwiGLU prologue into
    down (fused.gemv_rmsnorm / gemv_swiglu), against the same launches without
    prologues: what the fusion costs inside the GEMVs (the separate norm and
    SwiGLU kernels it removes are not counted here)."""
    from dequant_project_amd import fused

    gen = torch.Generator(device="cuda").manual_seed(20251205)
    gamma = torch.rand(HIDDEN, generator=gen, device="cuda", dtype=torch.float16) + 0.5
    ups = [torch.randn(1, INTER, generator=gen, device="cuda", dtype=torch.float16) for _ in stack]
    plain = step_launches(stack, xs, "decode")
    step_bytes = sum(launch_bytes(x, p) for _, x, p in plain)

    def run_plain():
        for _, x, p in plain:
            eng.gemv_group(x, p)

    def run_fused():
        for li, (layer, x) in enumerate(zip(stack, xs)):
            fused.gemv_rmsnorm(x["qkv"], gamma, 1e-5, [layer["q_proj"], layer["k_proj"], layer["v_proj"]])
            eng.gemv_group([x["o"]], [layer["o_proj"]])
            fused.gemv_rmsnorm(x["gate_up"], gamma, 1e-5, [layer["gate_proj"], layer["up_proj"]])
            fused.gemv_swiglu(x["down"], ups[li], layer["down_proj"])

    out = {}
    for name, fn in (("plain", run_plain), ("fused_prologues", run_fused)):
        graph = capture(torch, fn)
        ms, per = time_graph(torch, graph, steps, warmup)
        del graph
        out[name] = {"ms_per_step": ms, "step_ms": summarize(per), "us_per_layer": ms * 1e3 / len(stack),
                     "gbs": step_bytes / (ms * 1e-3) / 1e9}
    out["bytes_per_step"] = step_bytes
    return out


# a Llama-3-70B-shape stack in mixed precision
C5_LAYERS = 80
C5_HIDDEN, C5_KV, C5_INTER, C5_VOCAB = 8192, 1024, 28672, 128256


def c5_stack(torch, eng, steps, warmup, layers=C5_LAYERS):
    """80 layers of q/k/v/o in INT4 g128 asym and gate/up/down in INT2 g64
    asym, plus an INT8 per-channel sym lm_head 8192 -> 128256 (~25 GB
    packed), from seeded fp16 N(0, 0.02) weights quantized on the GPU one
    tensor at a time; x fp16 N(0, 1), batch 1. Timed as grouped launches of
    equal format and K ("stack") and as a decoder launches them ("decode":
    q|k|v, o, gate|up, down per layer, then the lm_head)."""
    from dequant_project_amd.packer import QuantConfig, quantize_tensor

    attn, mlp, head = QuantConfig(4, 128, False), QuantConfig(2, 64, False), QuantConfig(8, None, True)
    gen = torch.Generator(device="cuda").manual_seed(20251206)

    def q(n, k, cfg):
        w = torch.randn(n, k, generator=gen, device="cuda", dtype=torch.float16) * 0.02
        pw = quantize_tensor(w, cfg)
        del w
        return pw

    t0 = time.perf_counter()
    stack = []
    for _ in range(layers):
        stack.append({"q_proj": q(C5_HIDDEN, C5_HIDDEN, attn), "k_proj": q(C5_KV, C5_HIDDEN, attn),
                      "v_proj": q(C5_KV, C5_HIDDEN, attn), "o_proj": q(C5_HIDDEN, C5_HIDDEN, attn),
                      "gate_proj": q(C5_INTER, C5_HIDDEN, mlp), "up_proj": q(C5_INTER, C5_HIDDEN, mlp),
                      "down_proj": q(C5_HIDDEN, C5_INTER, mlp)})
    lm_head = q(C5_VOCAB, C5_HIDDEN, head)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    xs = [{"qkv": torch.randn(1, C5_HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
           "o": torch.randn(1, C5_HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
           "gate_up": torch.randn(1, C5_HIDDEN, generator=gen, device="cuda", dtype=torch.float16),
           "down": torch.randn(1, C5_INTER, generator=gen, device="cuda", dtype=torch.float16)} for _ in stack]
    x_head = torch.randn(1, C5_HIDDEN, generator=gen, device="cuda", dtype=torch.float16)

    launches = {}
    groups = {}
    for layer, x in zip(stack, xs):
        for role, names in GROUPS:
            for n in names:
                p = layer[n]
                groups.setdefault((p.config.bits, p.shape[1]), []).append((x[role], p))
    launches["stack"] = [([c[0] for c in items[i:i + 16]], [c[1] for c in items[i:i + 16]])
                         for items in groups.values() for i in range(0, len(items), 16)]
    launches["decode"] = [([x[role]] * len(names), [layer[n] for n in names])
                          for layer, x in zip(stack, xs) for role, names in GROUPS]
    for mode in launches:
        launches[mode].append(([x_head], [lm_head]))
    out = {"layers": layers, "build_s": build_s}
    for mode, ls in launches.items():
        step_bytes = sum(launch_bytes(x, p) for x, p in ls)

        def fn():
            for x, p in ls:
                eng.gemv_group(x, p)

        graph = capture(torch, fn)
        ms, per = time_graph(torch, graph, steps, warmup)
        del graph
        out[mode] = {"launches_per_step": len(ls), "bytes_per_step": step_bytes, "ms_per_step": ms,
                     "step_ms": summarize(per), "gbs": step_bytes / (ms * 1e-3) / 1e9,
                     "pct_peak": 100 * step_bytes / (ms * 1e-3) / 1e9 / PEAK_GBS,
                     "us_per_layer": ms * 1e3 / layers,
                     "kernel_instances": {k: len(v) for k, v in kernel_instances(eng, [(None, x, p) for x, p in ls]).items()}}
    del stack, lm_head, launches, groups
    torch.cuda.empty_cache()
    return out


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_m1_kernel_int4_c4_stack_traffic.md")


def profiled_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (copy-calibrated), or None if that summary is of
    another kernel."""
    try:
        text = open(TRAFFIC_PROFILE).read()
        rec = json.loads(text.split("```json", 1)[1].split("```", 1)[0])
    except (OSError, IndexError, ValueError):
        return None
    return rec["traffic_bytes_per_launch"] if rec.get("kernel") == kernel else None


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the sharding design is described in DESIGN.md", file=sys.stderr)
        return 2
    import torch

    from dequant_project_amd.packer import QuantConfig

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    eng = Engine(torch)
    torch.backends.cuda.matmul.allow_tf32 = False
    log(f"device: {torch.cuda.get_device_name(0)}  torch {torch.__version__}")

    if args.calibrate_copy:
        src = torch.empty(2 ** 28, dtype=torch.int32, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 1 GiB read + 1 GiB write, 3 times")
        del src, dst

    t0 = time.perf_counter()
    cfg, stack, xs = build_stack(torch, args.layers)
    torch.cuda.synchronize()
    log(f"built {args.layers}-layer INT4 stack in {time.perf_counter() - t0:.1f}s")

    modes = {}
    want = [m.strip() for m in args.modes.split(",") if m.strip()]
    if "stack" not in want:
        want.insert(0, "stack")
    for mode in want:
        launches, step_bytes, ms, per = run_mode(torch, eng, stack, xs, mode, args.steps, args.warmup)
        st = summarize(per)
        inst = kernel_instances(eng, launches)
        modes[mode] = {"launches_per_step": len(launches), "bytes_per_step": step_bytes, "ms_per_step": ms,
                       "step_ms": st, "gbs": step_bytes / (ms * 1e-3) / 1e9,
                       "us_per_layer": ms * 1e3 / args.layers,
                       "pct_peak": 100 * step_bytes / (ms * 1e-3) / 1e9 / PEAK_GBS,
                       "kernel_instances": {k: len(v) for k, v in inst.items()}}
        log(f"mode {mode}: {ms:.3f} ms/step  {modes[mode]['gbs']:.1f} GB/s  "
            f"{modes[mode]['us_per_layer']:.2f} us/layer  ({len(launches)} launches)")
        if mode == "stack":
            head_launches, head_bytes, head_ms, head_inst = launches, step_bytes, ms, inst

    # the stack step runs a single kernel instance: its mean launch duration is
    # the timed region over the launches in it (gaps between the 14 long
    # launches are included, a few percent)
    dominant = max(head_inst, key=lambda k: sum(head_inst[k]))
    n_dom = len(head_inst[dominant])
    bytes_per_launch = sum(head_inst[dominant]) / n_dom
    mean_us = head_ms * 1e3 / len(head_launches) if len(head_inst) == 1 else None
    achieved = bytes_per_launch / (mean_us * 1e-6) / 1e9 if mean_us else None
    if mean_us:
        log(f"dominant kernel {dominant}: {n_dom} launches/step, {bytes_per_launch / 1e6:.1f} MB/launch, "
            f"{mean_us:.2f} us/launch, {achieved:.1f} GB/s")
    else:
        log(f"dominant kernel {dominant}: {n_dom} launches/step, {bytes_per_launch / 1e6:.1f} MB/launch "
            f"(the step mixes {len(head_inst)} kernel instances: no per-launch duration)")
    traffic = profiled_traffic(dominant)
    roofline = {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBS, "unit": "GB/s",
                "frac": achieved / PEAK_GBS if achieved else None,
                "traffic": traffic, "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                                    "copy-calibrated; profiles/)", "kernel": dominant,
                "bytes_per_launch": bytes_per_launch, "mean_launch_us": mean_us, "launches_per_step": n_dom}

    # the same stack step in the other formats (sustained bandwidth of the
    # INT8 and INT2 kernels over the Llama-3-8B shapes)
    other_stacks = {}
    if not args.no_extra:
        for key, ocfg in [("INT8 per-channel sym", QuantConfig(8, None, True)),
                          ("INT2 g64 asym", QuantConfig(2, 64, False))]:
            _, ostack, oxs = build_stack(torch, args.layers, seed=20251202, cfg=ocfg)
            torch.cuda.synchronize()
            launches, step_bytes, ms, per = run_mode(torch, eng, ostack, oxs, "stack", args.steps, args.warmup)
            inst = kernel_instances(eng, launches)
            other_stacks[key] = {"launches_per_step": len(launches), "bytes_per_step": step_bytes,
                                 "ms_per_step": ms, "step_ms": summarize(per),
                                 "gbs": step_bytes / (ms * 1e-3) / 1e9, "us_per_layer": ms * 1e3 / args.layers,
                                 "pct_peak": 100 * step_bytes / (ms * 1e-3) / 1e9 / PEAK_GBS,
                                 "kernel_instances": {k: len(v) for k, v in inst.items()}}
            log(f"stack {key}: {ms:.3f} ms/step  {other_stacks[key]['gbs']:.1f} GB/s  "
                f"{other_stacks[key]['us_per_layer']:.2f} us/layer  ({len(launches)} launches)")
            del ostack, oxs, launches
            torch.cuda.empty_cache()

    # the same INT4 stack at the other batch sizes the benchmark configs name
    # (C4: M in {1, 2, 4, 8})
    batch_stacks = {}
    if not args.no_extra:
        gen = torch.Generator(device="cuda").manual_seed(20251203)
        for m in (2, 4, 8):
            mxs = make_xs(torch, args.layers, m, gen)
            launches, step_bytes, ms, per = run_mode(torch, eng, stack, mxs, "stack", args.steps, args.warmup)
            inst = kernel_instances(eng, launches)
            batch_stacks[f"M={m}"] = {"launches_per_step": len(launches), "bytes_per_step": step_bytes,
                                      "ms_per_step": ms, "step_ms": summarize(per),
                                      "gbs": step_bytes / (ms * 1e-3) / 1e9, "us_per_layer": ms * 1e3 / args.layers,
                                      "pct_peak": 100 * step_bytes / (ms * 1e-3) / 1e9 / PEAK_GBS,
                                      "kernel_instances": {k: len(v) for k, v in inst.items()}}
            log(f"stack INT4 M={m}: {ms:.3f} ms/step  {batch_stacks[f'M={m}']['gbs']:.1f} GB/s  "
                f"{batch_stacks[f'M={m}']['us_per_layer']:.2f} us/layer")
            del mxs, launches

    # the fused small GEMM over the stack (M > 8: the reference's dequantize +
    # F.linear path) and the decode launches with fused prologues
    gemm = {}
    prologue = None
    if not args.no_extra:
        for m in (16, 64):
            gemm[f"M={m}"] = gemm_stack(torch, stack, m, args.steps, args.warmup // 4)
            g = gemm[f"M={m}"]
            log(f"gemm_small stack M={m}: {g['ms_per_step']:.3f} ms/step  {g['gbs']:.1f} GB/s  "
                f"(dequantize + F.linear {g['dequantize_plus_linear_ms_per_step']:.3f} ms/step, "
                f"{g['speedup_vs_dequantize_plus_linear']:.2f}x)")
        prologue = prologue_decode(torch, eng, stack, xs, args.steps, args.warmup)
        log(f"decode launches: plain {prologue['plain']['us_per_layer']:.2f} us/layer, with fused prologues "
            f"{prologue['fused_prologues']['us_per_layer']:.2f} us/layer")

    c5 = None
    if not args.no_extra:
        c5 = c5_stack(torch, eng, args.steps, args.warmup // 4)
        log(f"C5 (Llama-3-70B shapes, INT4 attention / INT2 MLP / INT8 lm_head, {c5['stack']['bytes_per_step'] / 1e9:.2f} GB,"
            f" built in {c5['build_s']:.0f}s): stack {c5['stack']['ms_per_step']:.3f} ms/step "
            f"{c5['stack']['gbs']:.1f} GB/s {c5['stack']['us_per_layer']:.2f} us/layer; decode "
            f"{c5['decode']['ms_per_step']:.3f} ms/step {c5['decode']['gbs']:.1f} GB/s")

    extra = {}
    if not args.no_extra:
        for name, n, k, c, m in [("C1", 4096, 4096, QuantConfig(4, 128, False), 1),
                                 ("C2", 11008, 4096, QuantConfig(8, None, True), 1),
                                 ("C2_M4", 11008, 4096, QuantConfig(8, None, True), 4),
                                 ("C3", 4096, 11008, QuantConfig(2, 64, False), 1)]:
            key, res = single_config(torch, eng, name, n, k, c, m)
            extra[key] = res
            log(f"{key}: {res['us_per_call']:.2f} us/call ({res['gbs']:.0f} GB/s) in a graph of "
                f"{res['copies']} distinct copies")

    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        cpu = cpu_baseline(torch, stack)
        log(f"cpu baseline: {cpu['value']:.3f} GB/s on {cpu['cores']} threads ({time.perf_counter() - t0:.1f}s)")

    gbs = head_bytes / (head_ms * 1e-3) / 1e9
    line = {
        "metric": METRIC, "value": gbs, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head_ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int4 codes -> fp16 (q-z), fp16 x fp16 products, fp32 accumulate",
        "data": "synthetic (seeded fp16 N(0,0.02) weights quantized on the GPU; fp16 N(0,1) activations)",
        "config": {"workload": "C4: Llama-3-8B decoder linear set (32 layers x q,k,v,o,gate,up,down), "
                               "INT4 g128 asym, M=1",
                   "layers": args.layers, "batch": 1, "bytes_per_step": head_bytes,
                   "launches_per_step": len(head_launches),
                   "grouping": "stack: launches of up to 16 independent GEMVs of equal K"},
        "pct_of_peak": 100 * gbs / PEAK_GBS,
        "us_per_layer": head_ms * 1e3 / args.layers,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "modes": modes,
        "other_format_stacks": other_stacks,
        "batch_stacks": batch_stacks,
        "gemm_small_stacks": gemm,
        "decode_with_fused_prologues": prologue,
        "c5_llama3_70b_stack": c5,
        "single_configs": extra,
    }
    print(json.dumps(line, default=lambda o: sorted(o) if isinstance(o, set) else str(o)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
