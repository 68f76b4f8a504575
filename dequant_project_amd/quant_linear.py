"""QuantLinear: an nn.Linear drop-in whose weight exists only in packed form.

Public surface of the reference's dequant/quant_linear.py (MAX_M :39, PROJ
:44, _get_ext :49-69, gemv :72-82, dequantize_cuda :85-93, QuantLinear
:96-140, quantize_model :143-162), backed by the gfx950 engine:

  M <= MAX_M   the fused dequant + GEMV kernel (dequant_cuda.gemv): codes are
               unpacked in registers, nothing is materialized. The decode path.
  M <= MAX_M_GEMM, where uses_gemm_small (no reference counterpart): the
               fused small GEMM (dequant_cuda.gemm_small): the reference's
               M > MAX_M product, x @ dequantize(W)^T over the same fp16
               weight, formed in registers in one pass over the packed bytes
               instead of materializing it; equal to the path below up to the
               order of the fp32 summation.
  otherwise    dequant_cuda.dequantize materializes the fp16 [N, K] weight
               (bit-exact with packer.dequantize) and F.linear does the GEMM
               (the reference's branch for every M > MAX_M).

Both branches launch on the current HIP stream and never synchronize, so a
forward pass can be captured into a HIP graph (torch.cuda.CUDAGraph). There is
no CPU or pure-torch fallback: without the built extension `_get_ext()`
raises ImportError.
"""

import torch
import torch.nn.functional as F
from torch import nn

from . import _native
from .packer import PackedWeight, QuantConfig, quantize_tensor

# Largest batch the fused kernel handles; above it the dequantize fallback runs.
MAX_M = 8

# Largest batch the fused small GEMM takes (batched decode, short prefills);
# above it dequantize + F.linear runs. No reference counterpart.
MAX_M_GEMM = 64

# Measured on MI355X against dequantize + F.linear over the Llama-3-8B
# projection shapes: the fused small GEMM is faster at every batch of 9..64
# rows, at 33..64 rows by 1.5-2.4x across INT4 / INT8 / INT2 formats on the
# 4096 x 4096, 14336 x 4096 and 4096 x 14336 weights (the column walk), so
# the whole range takes it.


def uses_gemm_small(m, n, k, cfg=None, x=None):
    """Whether QuantLinear runs the fused small GEMM for m rows of an [n, k] weight.

    Batches of 9..64 rows take it under the GEMV kernels' operand rules:
    group_size a multiple of 128/bits codes (one 16-byte chunk per group at
    least; INT2 g32 is excluded) and x 16-byte aligned. Inputs outside them
    take the reference's dequantize + F.linear path, which has neither
    restriction.
    """
    if not MAX_M < m <= MAX_M_GEMM:
        return False
    if cfg is not None and cfg.effective_group_size(k) % (128 // cfg.bits) != 0:
        return False
    if x is not None and x.data_ptr() % 16 != 0:
        return False
    return True

# The projections of a Llama-style decoder layer that quantize_model replaces.
PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def _get_ext():
    """The `dequant_cuda` extension module; ImportError with a build hint if absent."""
    return _native.ext()


def gemv(x, pw: PackedWeight):
    """y = x @ W^T with W packed. x fp16 [..., K] -> y fp16 [..., N]."""
    n, k = pw.shape
    cfg = pw.config
    x2 = x.reshape(-1, k).contiguous()
    y = _get_ext().gemv(x2, pw.qweight, pw.scales, pw.zeros, cfg.bits,
                        cfg.effective_group_size(k), cfg.symmetric,
                        cfg.layout == "interleaved")
    return y.view(*x.shape[:-1], n)


def gemv_grouped(xs, pws):
    """Several y_i = x_i @ W_i^T in ONE kernel launch (no reference counterpart).

    All weights must share bits / symmetry / layout and all x_i the same
    number of rows (at most MAX_M); up to 16 problems. Results match calling
    gemv() per problem up to fp32 rounding of the split-K partial sums (the
    launch geometry depends on the whole group) and are deterministic for a
    given group. This is the grouped decode launch: q|k|v (same x) or gate|up
    of a Llama layer.
    """
    if not pws:
        return []
    cfg0 = pws[0].config
    if any(pw.config.bits != cfg0.bits or pw.config.symmetric != cfg0.symmetric
           or pw.config.layout != cfg0.layout for pw in pws):
        raise ValueError("gemv_grouped: all weights must share bits, symmetric and layout")
    x2s = [x.reshape(-1, pw.shape[1]).contiguous() for x, pw in zip(xs, pws)]
    ys = _get_ext().gemv_batched(
        x2s, [pw.qweight for pw in pws], [pw.scales for pw in pws], [pw.zeros for pw in pws],
        cfg0.bits, [pw.config.effective_group_size(pw.shape[1]) for pw in pws], cfg0.symmetric,
        cfg0.layout == "interleaved")
    return [y.view(*x.shape[:-1], pw.shape[0]) for y, x, pw in zip(ys, xs, pws)]


def gemm_small(x, pw: PackedWeight):
    """y = x @ dequantize(W)^T for up to MAX_M_GEMM rows, in one pass over the
    packed weight (no reference counterpart; see the module docstring)."""
    n, k = pw.shape
    cfg = pw.config
    x2 = x.reshape(-1, k).contiguous()
    y = _get_ext().gemm_small(x2, pw.qweight, pw.scales, pw.zeros, cfg.bits,
                              cfg.effective_group_size(k), cfg.symmetric,
                              cfg.layout == "interleaved")
    return y.view(*x.shape[:-1], n)


def dequantize_cuda(pw: PackedWeight):
    """fp16 [N, K] on the GPU, bit-exact with packer.dequantize."""
    n, k = pw.shape
    cfg = pw.config
    return _get_ext().dequantize(pw.qweight, pw.scales, pw.zeros, cfg.bits,
                                 cfg.effective_group_size(k), cfg.symmetric,
                                 cfg.layout == "interleaved", k)


class QuantLinear(nn.Module):
    """nn.Linear replacement holding only qweight / scales / zeros (+ bias) buffers.

    There is deliberately no `.weight`, so nothing can fall back to an fp16
    matmul over a full-size weight.
    """

    def __init__(self, pw: PackedWeight, bias=None):
        super().__init__()
        self.out_features, self.in_features = pw.shape
        self.config = pw.config
        self.register_buffer("qweight", pw.qweight)
        self.register_buffer("scales", pw.scales)
        self.register_buffer("zeros", pw.zeros)
        self.register_buffer("bias", bias)

    @classmethod
    def from_linear(cls, linear: nn.Linear, cfg: QuantConfig):
        pw = quantize_tensor(linear.weight.data, cfg)
        bias = None if linear.bias is None else linear.bias.data.to(torch.float16)
        return cls(pw, bias)

    def _packed(self):
        # Rebuilt on every call so that .to() / .cuda() moves stay visible.
        return PackedWeight(qweight=self.qweight, scales=self.scales, zeros=self.zeros,
                            config=self.config, shape=(self.out_features, self.in_features))

    def forward(self, x):
        pw = self._packed()
        m = x.numel() // self.in_features
        if m <= MAX_M:
            y = gemv(x, pw)
        elif uses_gemm_small(m, self.out_features, self.in_features, self.config,
                             x.reshape(-1, self.in_features).contiguous()):
            y = gemm_small(x, pw)
        else:
            y = F.linear(x, dequantize_cuda(pw))
        if self.bias is not None:
            y = y + self.bias
        return y

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, config={self.config}")


def quantize_model(model, cfg: QuantConfig, names=PROJ):
    """Swap every nn.Linear whose leaf name is in `names` for a QuantLinear, in place.

    Returns {"replaced", "packed_bytes", "fp16_bytes"}.
    """
    replaced = packed_bytes = fp16_bytes = 0
    for path, mod in list(model.named_modules()):
        leaf = path.rsplit(".", 1)[-1]
        if leaf not in names or not isinstance(mod, nn.Linear):
            continue
        parent = model.get_submodule(path.rsplit(".", 1)[0] if "." in path else "")
        ql = QuantLinear.from_linear(mod, cfg)
        setattr(parent, leaf, ql)
        replaced += 1
        packed_bytes += ql._packed().nbytes
        fp16_bytes += mod.weight.numel() * 2
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return {"replaced": replaced, "packed_bytes": packed_bytes, "fp16_bytes": fp16_bytes}
