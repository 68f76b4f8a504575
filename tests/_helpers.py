"""Shared test helpers: seeded synthetic weights and oracle glue (CPU side)."""

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_LIB = ROOT / "oracle" / "_build" / "libdq_oracle.so"


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def gauss_weight(n, k, seed, std=0.02):
    """fp16 N(0, std) weight [N, K] (the configs' synthetic weights)."""
    return (rng(seed).standard_normal((n, k), dtype=np.float32) * std).astype(np.float16)


def skew_weight(n, k, seed):
    """All-positive U(2, 2.5): large negative zero points (test_dequant_kernel.py:68-70)."""
    return (rng(seed).random((n, k), dtype=np.float32) * 0.5 + 2.0).astype(np.float16)


def outlier_weight(n, k, seed, std=0.02, frac=1e-3, sigmas=10.0):
    """N(0, std) with a seeded `frac` of entries set to +-sigmas*std (config C3)."""
    g = rng(seed)
    w = g.standard_normal((n, k), dtype=np.float32) * std
    cnt = max(1, int(round(frac * n * k)))
    idx = g.choice(n * k, cnt, replace=False)
    w.reshape(-1)[idx] = np.where(g.random(cnt) < 0.5, -sigmas * std, sigmas * std)
    return w.astype(np.float16)


def activations(m, k, seed):
    """fp16 N(0, 1) activations [M, K]."""
    return rng(seed).standard_normal((m, k), dtype=np.float32).astype(np.float16)


def oracle_lib():
    """ctypes handle on the C oracle, building it with oracle/Makefile if needed."""
    if not ORACLE_LIB.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)
    lib = ctypes.CDLL(str(ORACLE_LIB))
    P, I, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    lib.dqo_unpack.argtypes = [P, P, I64, I64, I, I]
    lib.dqo_dequantize.argtypes = [P, P, P, P, I64, I64, I, I64, I, I]
    lib.dqo_exact_weight.argtypes = [P, P, P, P, I64, I64, I, I64, I, I]
    lib.dqo_gemv_ref.argtypes = [P, P, P, P, I64, I64, I64]
    lib.dqo_f32_to_f16_array.argtypes = [P, P, I64]
    lib.dqo_f32_to_f16.argtypes = [ctypes.c_float]
    lib.dqo_f32_to_f16.restype = ctypes.c_uint16
    lib.dqo_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.dqo_f16_to_f32.restype = ctypes.c_float
    return lib


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def golden():
    return np.load(ROOT / "tests" / "golden" / "packer_golden.npz")


def golden_tag(bits, gs, sym, layout):
    return f"b{bits}_g{'pc' if gs is None else gs}_{'sym' if sym else 'asym'}_{layout[:3]}"


GOLDEN_CASES = [(b, g, s, l) for b in (2, 4, 8) for g in (32, 64, 128, None)
                for s in (True, False) for l in ("sequential", "interleaved")]
