"""Offline quantizer and the packed INT2/INT4/INT8 weight format.

Same public API and the same bytes as the reference's dequant/packer.py
(QuantConfig :44-78, PackedWeight :81-96, quantize :99-143, pack :146-161,
unpack :164-174, dequantize :177-189, quantize_tensor :192-201), so packed
weights made by either side are interchangeable. The engine's kernels read
this format directly:

  * a weight is [N, K]; the GEMV reduces over K; groups of `group_size`
    consecutive K entries share one fp16 scale (and zero point);
  * codes are unsigned; symmetric quantization stores code + 2^(bits-1);
  * a 32-bit word holds 32/bits codes; "sequential" puts logical code i at bit
    offset bits*i, "interleaved" puts logical INTERLEAVE[bits][s] in slot s;
  * qweight is int32 carrying the uint32 bit pattern.

The functions use plain torch ops and run on whichever device the input lives
on (the benchmark quantizes its multi-GB synthetic stacks on the GPU). The
quantizer's arithmetic steps follow the reference's exactly -- same fp32
expressions, half-to-even rounding, 0 -> 1 scale substitution before the fp16
rounding, unclamped fp16 zero points -- because identical codes are part of the
drop-in contract; tests/golden/packer_golden.npz pins that bit for bit.
"""

from dataclasses import dataclass

import torch

# Slot -> logical code for the interleaved layout (the format's own table).
_INTERLEAVE = {
    4: [0, 2, 4, 6, 1, 3, 5, 7],
    2: [0, 4, 8, 12, 1, 5, 9, 13, 2, 6, 10, 14, 3, 7, 11, 15],
    8: [0, 2, 1, 3],
}


@dataclass(frozen=True)
class QuantConfig:
    bits: int = 4
    group_size: int | None = 128   # None: one scale per output row (per-channel)
    symmetric: bool = True
    layout: str = "sequential"     # or "interleaved"

    def __post_init__(self):
        if self.bits not in (2, 4, 8):
            raise ValueError(f"bits must be 2, 4 or 8, got {self.bits}")
        if self.layout not in ("sequential", "interleaved"):
            raise ValueError(f"unknown layout: {self.layout!r}")
        if self.group_size is not None and self.group_size <= 0:
            raise ValueError("group_size must be positive or None")

    @property
    def per_pack(self):
        """Codes per 32-bit word."""
        return 32 // self.bits

    @property
    def qmax(self):
        """Largest unsigned code."""
        return (1 << self.bits) - 1

    @property
    def bias(self):
        """Offset added to symmetric codes."""
        return 1 << (self.bits - 1)

    def groups_for(self, k):
        return 1 if self.group_size is None else k // self.group_size

    def effective_group_size(self, k):
        return k if self.group_size is None else self.group_size


@dataclass
class PackedWeight:
    """Packed codes plus the metadata that reconstructs the weight."""

    qweight: torch.Tensor          # int32 (uint32 bits) [N, K // per_pack]
    scales: torch.Tensor           # fp16 [N, n_groups]
    zeros: torch.Tensor | None     # fp16 [N, n_groups] when asymmetric
    config: QuantConfig
    shape: tuple                   # (N, K)

    @property
    def nbytes(self):
        total = self.qweight.numel() * 4 + self.scales.numel() * 2
        if self.zeros is not None:
            total += self.zeros.numel() * 2
        return total


def _slot_order(cfg):
    return _INTERLEAVE[cfg.bits] if cfg.layout == "interleaved" else list(range(cfg.per_pack))


def quantize(w, cfg: QuantConfig):
    """[N, K] weight -> (codes int32 [N, K] in [0, qmax], scales fp16, zeros fp16 | None)."""
    if w.dim() != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(w.shape)}")
    n, k = w.shape
    gs = cfg.effective_group_size(k)
    if k % gs:
        raise ValueError(f"K={k} is not divisible by group_size={gs}")

    grouped = w.float().reshape(n, k // gs, gs)
    if cfg.symmetric:
        step = grouped.abs().amax(dim=-1, keepdim=True) / (cfg.bias - 1)
        step = torch.where(step == 0, torch.ones_like(step), step)
        step = step.to(torch.float16).float()       # codes are chosen against the stored fp16 scale
        codes = torch.round(grouped / step) + cfg.bias
        zero = None
    else:
        hi = grouped.amax(dim=-1, keepdim=True)
        lo = grouped.amin(dim=-1, keepdim=True)
        step = (hi - lo) / cfg.qmax
        step = torch.where(step == 0, torch.ones_like(step), step)
        step = step.to(torch.float16).float()
        zero = torch.round(-lo / step)              # not clamped; stored as fp16
        codes = torch.round(grouped / step) + zero

    codes = codes.clamp_(0, cfg.qmax).to(torch.int32).reshape(n, k)
    scales = step.reshape(n, -1).to(torch.float16)
    zeros = None if zero is None else zero.reshape(n, -1).to(torch.float16)
    return codes, scales, zeros


def pack(q, cfg: QuantConfig):
    """Unsigned codes [N, K] -> int32 words [N, K // per_pack] (uint32 bit pattern)."""
    n, k = q.shape
    per = cfg.per_pack
    if k % per:
        raise ValueError(f"K={k} is not divisible by {per} values per word")
    lanes = q.reshape(n, k // per, per)
    words = torch.zeros(n, k // per, dtype=torch.int64, device=q.device)
    for slot, logical in enumerate(_slot_order(cfg)):
        words |= (lanes[:, :, logical].to(torch.int64) & cfg.qmax) << (cfg.bits * slot)
    return words.to(torch.int32)     # int64 -> int32 keeps the low 32 bits


def unpack(packed, cfg: QuantConfig, k):
    """int32 words [N, K // per_pack] -> unsigned codes int32 [N, K]."""
    n = packed.shape[0]
    per = cfg.per_pack
    words = packed.to(torch.int64) & 0xFFFFFFFF
    codes = torch.empty(n, k // per, per, dtype=torch.int32, device=packed.device)
    for slot, logical in enumerate(_slot_order(cfg)):
        codes[:, :, logical] = ((words >> (cfg.bits * slot)) & cfg.qmax).to(torch.int32)
    return codes.reshape(n, k)


def dequantize(pw: PackedWeight):
    """fp16 [N, K] = fp16((code - offset) * scale), computed in fp32."""
    cfg = pw.config
    n, k = pw.shape
    gs = cfg.effective_group_size(k)
    q = unpack(pw.qweight, cfg, k).reshape(n, k // gs, gs).float()
    offset = cfg.bias if cfg.symmetric else pw.zeros.float().unsqueeze(-1)
    return ((q - offset) * pw.scales.float().unsqueeze(-1)).reshape(n, k).to(torch.float16)


def quantize_tensor(w, cfg: QuantConfig) -> PackedWeight:
    """quantize() then pack() into a PackedWeight."""
    q, scales, zeros = quantize(w, cfg)
    return PackedWeight(qweight=pack(q, cfg), scales=scales, zeros=zeros, config=cfg,
                        shape=tuple(w.shape))
