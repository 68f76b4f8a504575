"""Write the golden vectors for the packed format (run in the survey container only).

The reference's quantizer (dequant/packer.py:99-143, quantize_tensor :192-201)
is the one function on this path that no closed form pins bit for bit: fp32
division order, half-to-even ties, the 0 -> 1 scale substitution before the
fp16 rounding, and unclamped fp16 zero-points all shape its output. So this
script imports the reference's own packer.py from /root/reference, runs it on
small deterministic inputs, and stores inputs and outputs as data:

  tests/golden/packer_golden.npz
    w16                 uint16 [8, 256]  fp16 bit patterns of the input weight
    <tag>/qweight       int32  packed words     (packer.quantize_tensor)
    <tag>/scales        uint16 fp16 bits
    <tag>/zeros         uint16 fp16 bits (asymmetric tags only)
    <tag>/codes         int32  [8, 256]         (packer.unpack)
    <tag>/deq           uint16 fp16 bits [8, 256] (packer.dequantize)
  with <tag> = b{bits}_g{group or 'pc'}_{sym|asym}_{seq|int}.

Inputs are generated with numpy's PCG64 (seed 20251201), not torch's RNG, so
they are reproducible anywhere. The reference never leaves this container:
only the vectors are committed. Run:  python tests/golden/make_golden.py
"""

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

REF_PACKER = Path("/root/reference/dequant/packer.py")
OUT = Path(__file__).resolve().parent / "packer_golden.npz"

BITS = (2, 4, 8)
GROUPS = (32, 64, 128, None)
LAYOUTS = ("sequential", "interleaved")


def make_weight():
    """[8, 256] fp16 rows covering the quantizer's edge cases."""
    rng = np.random.Generator(np.random.PCG64(20251201))
    n, k = 8, 256
    w = np.zeros((n, k), dtype=np.float32)
    w[0] = rng.standard_normal(k) * 0.02                        # Llama-like
    w[1] = rng.standard_normal(k) * 0.02
    w[2] = rng.uniform(2.0, 2.5, k)                              # skewed: negative zero-points
    w[3] = 0.0                                                   # all-zero row: scale 0 -> 1
    w[4] = 0.37                                                  # constant row
    w[5] = rng.standard_normal(k) * 0.02                         # outliers at +-10 sigma
    idx = rng.choice(k, 6, replace=False)
    w[5, idx] = np.where(rng.random(6) < 0.5, -0.2, 0.2)
    w[6] = (rng.integers(-16, 17, k) * 0.5) * 0.0625             # many exact half-step ties
    w[7] = rng.standard_normal(k) * 3.0                          # wide range, large zero-points
    w[7, ::37] = 1e-7                                            # fp16 subnormal entries
    return w.astype(np.float16)


def tag(bits, gs, sym, layout):
    return f"b{bits}_g{'pc' if gs is None else gs}_{'sym' if sym else 'asym'}_{layout[:3]}"


def main():
    spec = importlib.util.spec_from_file_location("ref_packer", REF_PACKER)
    ref = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(ref)

    w16 = make_weight()
    wt = torch.from_numpy(w16.copy())
    out = {"w16": w16.view(np.uint16)}
    for bits in BITS:
        for gs in GROUPS:
            for sym in (True, False):
                for layout in LAYOUTS:
                    cfg = ref.QuantConfig(bits, gs, sym, layout)
                    pw = ref.quantize_tensor(wt, cfg)
                    t = tag(bits, gs, sym, layout)
                    out[f"{t}/qweight"] = pw.qweight.numpy().astype(np.int32)
                    out[f"{t}/scales"] = pw.scales.numpy().view(np.uint16)
                    if pw.zeros is not None:
                        out[f"{t}/zeros"] = pw.zeros.numpy().view(np.uint16)
                    out[f"{t}/codes"] = ref.unpack(pw.qweight, cfg, w16.shape[1]).numpy()
                    out[f"{t}/deq"] = ref.dequantize(pw).numpy().view(np.uint16)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    sys.exit(main())
