"""numpy restatement of the activation ops the fused prologues replace -- TEST ORACLE.

Test infrastructure only (see oracle/__init__.py). The reference's decode path
runs these ops as separate modules in front of its QuantLinear projections
(Hugging Face Llama, which its bench.py:88-174 loads; the fusion is the
reference's planned next step, MODEL_SELECTION.md:211-218). The module code
they restate is third-party: transformers' LlamaRMSNorm.forward and
LlamaMLP.forward (transformers 5.15.0 in this image, models/llama/
modeling_llama.py):

  rmsnorm_fp16   LlamaRMSNorm on fp16 activations: x in fp32, variance =
                 mean(x^2), x * rsqrt(variance + eps) rounded to fp16, times
                 the fp16 weight (an fp16 product);
  swiglu_fp16    act_fn(gate) * up with act_fn = SiLU on fp16 tensors: silu in
                 fp32 rounded to fp16, times up (an fp16 product);
  rmsnorm64 / swiglu64  the same maps in fp64 (the exact values the fused
                 kernels approximate).

Parity pinning (tests/test_prologue_oracle.py): closed forms (a constant
vector normalizes to sign * gamma; scale invariance with eps = 0; silu(g) =
g * logistic(g) against scipy.special.expit) and the transformers modules
themselves run on CPU fp16 tensors (rmsnorm_fp16 within one fp16 ulp: the
fp32 mean's summation order is the only freedom; swiglu_fp16 within two, where
an fp32 silu value sits at an fp16 rounding tie).
"""

import numpy as np


def rmsnorm64(x, gamma, eps):
    """x / sqrt(mean(x^2) + eps) * gamma over the last axis, in fp64."""
    x64 = np.asarray(x, dtype=np.float64)
    r = 1.0 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)
    return x64 * r * np.asarray(gamma, dtype=np.float64)


def rmsnorm_fp16(x, gamma, eps):
    """LlamaRMSNorm.forward on fp16 input: returns fp16."""
    x32 = np.asarray(x, dtype=np.float16).astype(np.float32)
    var = np.mean(x32 * x32, axis=-1, keepdims=True, dtype=np.float32)
    h16 = (x32 * (np.float32(1.0) / np.sqrt(var + np.float32(eps)))).astype(np.float16)
    return (np.asarray(gamma, dtype=np.float16).astype(np.float32) * h16.astype(np.float32)).astype(np.float16)


def silu64(g):
    g64 = np.asarray(g, dtype=np.float64)
    return g64 / (1.0 + np.exp(-g64))


def swiglu64(gate, up):
    """silu(gate) * up in fp64."""
    return silu64(gate) * np.asarray(up, dtype=np.float64)


def swiglu_fp16(gate, up):
    """SiLU(gate) * up on fp16 tensors: returns fp16."""
    g32 = np.asarray(gate, dtype=np.float16).astype(np.float32)
    with np.errstate(over="ignore"):
        s16 = (g32 / (np.float32(1.0) + np.exp(-g32))).astype(np.float16)
    return (s16.astype(np.float32) * np.asarray(up, dtype=np.float16).astype(np.float32)).astype(np.float16)
