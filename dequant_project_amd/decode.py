"""End-to-end decode on a locally constructed Llama, with QuantLinear projections.

The reference measures decode latency on Hugging Face models loaded by name
(dequant/bench.py:88-174, `AutoModelForCausalLM.from_pretrained`). Nothing is
downloaded here: the model is built from a `LlamaConfig` (shape presets
below, e.g. Llama-3-8B's), its weights are seeded random fp16, and
`quantize_model` swaps the seven projections of every layer for QuantLinear
(the engine's kernels: fused GEMV for a decode step). Attention, norms,
embeddings and the fp16 lm_head run on PyTorch.

One decode step is timed at a fixed context length, the reference's
discipline (dequant/bench.py:84-170):
  * the static KV cache holds exactly seq_len slots and its write counters
    are rewound after every step, so each step sees the same context;
  * three numbers per step: host_ms (Python returns, no sync), gpu_ms (HIP
    events around the step) and total_ms (with the sync);
  * modes: "eager" (the module call) and "graph" (the step captured into one
    HIP graph and replayed: what the GPU itself needs per token).

  python -m dequant_project_amd.decode --preset llama3-8b --seq-lens 128,1024
"""

import argparse
import json
import statistics
import sys
import time

import torch

from . import byte_model
from .packer import QuantConfig
from .quant_linear import QuantLinear, quantize_model

# Shapes of the models the benchmark configurations name (BASELINE.json C4, C5).
PRESETS = {
    "llama3-8b": dict(hidden_size=4096, intermediate_size=14336, num_hidden_layers=32, num_attention_heads=32,
                      num_key_value_heads=8, vocab_size=128256, rope_theta=500000.0),
    "llama3-70b": dict(hidden_size=8192, intermediate_size=28672, num_hidden_layers=80, num_attention_heads=64,
                       num_key_value_heads=8, vocab_size=128256, rope_theta=500000.0),
    # small shapes for tests
    "tiny": dict(hidden_size=256, intermediate_size=768, num_hidden_layers=2, num_attention_heads=4,
                 num_key_value_heads=2, vocab_size=512, rope_theta=10000.0),
}


def llama_config(preset, max_positions=4096, **overrides):
    from transformers import LlamaConfig

    kw = dict(PRESETS[preset])
    kw.update(overrides)
    return LlamaConfig(max_position_embeddings=max_positions, tie_word_embeddings=False, attn_implementation="sdpa",
                       **kw)


def build_llama(preset="llama3-8b", seed=0, device="cuda", dtype=torch.float16, std=0.02, **overrides):
    """A random-init LlamaForCausalLM of the preset's shape (no download)."""
    from transformers import LlamaForCausalLM

    cfg = llama_config(preset, **overrides)
    torch.manual_seed(seed)
    with torch.device(device):
        prev = torch.get_default_dtype()
        torch.set_default_dtype(dtype)
        try:
            model = LlamaForCausalLM(cfg)
        finally:
            torch.set_default_dtype(prev)
    gen = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        for p in model.parameters():
            if p.dim() >= 2:
                p.normal_(0.0, std, generator=gen)  # N(0, 0.02), the benchmark configs' weights
    return model.eval()


def summarize(samples):
    s = sorted(samples)
    n = len(s)
    return {"median": statistics.median(s), "p25": s[n // 4], "p75": s[(3 * n) // 4], "min": s[0], "max": s[-1],
            "n": n}


def _rewind(cache, pos):
    for layer in cache.layers:
        layer.cumulative_length.fill_(pos)


def decode_step_fn(model, seq_len, device="cuda"):
    """(step, restore, logits): one decode step at context seq_len on a static cache."""
    from transformers import StaticCache

    pos = seq_len - 1
    cache = StaticCache(config=model.config, max_cache_len=seq_len)
    ids = torch.randint(0, model.config.vocab_size, (1, pos), device=device,
                        generator=torch.Generator(device=device).manual_seed(seq_len))
    with torch.no_grad():
        model(input_ids=ids, past_key_values=cache, cache_position=torch.arange(pos, device=device), use_cache=True)
    token = torch.tensor([[int(ids[0, -1])]], device=device)
    cache_position = torch.tensor([pos], device=device)
    out = {}

    def step():
        # transformers' StaticLayer.update takes its write slot from a counter
        # that every step advances, not from cache_position; rewinding it first
        # keeps each step (eager or replayed) at slot seq_len - 1, inside the
        # seq_len-slot buffer, whatever ran before
        _rewind(cache, pos)
        with torch.no_grad():
            out["logits"] = model(input_ids=token, past_key_values=cache, cache_position=cache_position,
                                  use_cache=True).logits

    def restore():
        _rewind(cache, pos)

    return step, restore, out


def time_decode(model, seq_len, mode="graph", warmup=10, iters=30, device="cuda"):
    step, restore, out = decode_step_fn(model, seq_len, device)
    if mode == "graph":
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                step()
                restore()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        restore()
        with torch.cuda.graph(graph):
            step()
        run = graph.replay
    elif mode == "eager":
        run = step
    else:
        raise ValueError(f"unknown mode {mode!r}")
    for _ in range(warmup):
        run()
        restore()
    torch.cuda.synchronize()
    host, gpu, total = [], [], []
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(iters):
        t0 = time.perf_counter()
        a.record()
        run()
        b.record()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        host.append((t1 - t0) * 1e3)
        gpu.append(a.elapsed_time(b))
        total.append((t2 - t0) * 1e3)
        restore()
    return {"host_ms": summarize(host), "gpu_ms": summarize(gpu), "total_ms": summarize(total)}, out


def quantized_bytes_per_token(model, seq_len):
    """Bytes one decode step reads: packed projections + fp16 rest + KV cache."""
    packed = sum(m._packed().nbytes for m in model.modules() if isinstance(m, QuantLinear))
    spec = byte_model.spec_from_hf_config(model.config.to_dict())
    fp16_total = byte_model.decode_bytes(spec, seq_len, weight_dtype="fp16")
    quant_fp16 = sum(m.in_features * m.out_features * 2 for m in model.modules() if isinstance(m, QuantLinear))
    return fp16_total["total"] - quant_fp16 + packed


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--preset", default="llama3-8b", choices=sorted(PRESETS))
    ap.add_argument("--layers", type=int, default=None, help="override the layer count")
    ap.add_argument("--bits", type=int, default=4)
    ap.add_argument("--group-size", type=int, default=128, help="0 = per-channel")
    ap.add_argument("--symmetric", action="store_true")
    ap.add_argument("--seq-lens", default="128,1024")
    ap.add_argument("--modes", default="graph,eager")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--iters", type=int, default=30)
    ap.add_argument("--fp16-baseline", action="store_true", help="also time the unquantized fp16 model")
    ap.add_argument("--fused", action="store_true",
                    help="also time the quantized model with fused RMSNorm / SwiGLU prologues (fused.fuse_llama)")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("decode.py needs a GPU", file=sys.stderr)
        return 1
    over = {} if args.layers is None else {"num_hidden_layers": args.layers}
    seq_lens = [int(s) for s in args.seq_lens.split(",") if s]
    modes = [m for m in args.modes.split(",") if m]
    model = build_llama(args.preset, **over)
    rec = {"preset": args.preset, "layers": model.config.num_hidden_layers, "device": torch.cuda.get_device_name(0),
           "data": "synthetic: random-init fp16 N(0, 0.02) weights (no checkpoint)", "rows": []}
    if args.fp16_baseline:
        spec = byte_model.spec_from_hf_config(model.config.to_dict())
        for n in seq_lens:
            t, _ = time_decode(model, n, "graph", args.warmup, args.iters)
            b = byte_model.decode_bytes(spec, n, weight_dtype="fp16")["total"]
            rec["rows"].append({"weights": "fp16", "seq_len": n, "mode": "graph", **t, "bytes_per_token": b,
                                "gbs": b / (t["gpu_ms"]["median"] * 1e-3) / 1e9})
            print(json.dumps(rec["rows"][-1]["gpu_ms"]), file=sys.stderr)
    cfg = QuantConfig(args.bits, args.group_size or None, args.symmetric, "sequential")
    stats = quantize_model(model, cfg)
    rec["quant"] = {"config": repr(cfg), **stats}
    for n in seq_lens:
        _time_rows(rec, model, cfg, n, modes, args, "unfused")
    if args.fused:
        from .fused import fuse_llama

        rec["fused"] = fuse_llama(model)  # in place, after the unfused rows
        for n in seq_lens:
            _time_rows(rec, model, cfg, n, modes, args, "fused")
    print(json.dumps(rec))
    return 0


def _time_rows(rec, model, cfg, n, modes, args, label):
    b = quantized_bytes_per_token(model, n)
    for mode in modes:
        t, _ = time_decode(model, n, mode, args.warmup, args.iters)
        row = {"weights": repr(cfg), "prologues": label, "seq_len": n, "mode": mode, **t, "bytes_per_token": b,
               "gbs": b / (t["gpu_ms"]["median"] * 1e-3) / 1e9,
               "us_per_token": t["gpu_ms" if mode == "graph" else "total_ms"]["median"] * 1e3}
        rec["rows"].append(row)
        print(f"{cfg.bits}-bit {label} seq {n} {mode}: {row['us_per_token']:.0f} us/token "
              f"(gpu {t['gpu_ms']['median']:.3f} ms, {row['gbs']:.0f} GB/s)", file=sys.stderr)


if __name__ == "__main__":
    sys.exit(main())
