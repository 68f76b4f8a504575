"""numpy restatement of the reference's packed INT2/4/8 format -- TEST ORACLE.

Test infrastructure only (see oracle/__init__.py). Each function follows the
reference file:line named in its docstring; arithmetic is done in the same
precision as the reference's torch code (fp32, round-half-to-even, fp16 RNE
casts), so outputs are bit-identical to the reference for the same inputs.

Parity pinning (tests/test_oracle.py):
  pack / unpack      known-answer words derived from the interleave tables,
                     brute force over every code value, roundtrip.
  quantize           golden vectors written by importing the reference's own
                     packer.py (tests/golden/make_golden.py), plus the
                     reference tests' invariants (error bound, monotonicity).
  dequantize         golden vectors + closed form on hand-picked codes.
  exact_weight/gemv  fp64 brute force on tiny shapes, linearity, the
                     negative control of scripts/test_dequant_kernel.py:194-217.
"""

import numpy as np

# dequant/packer.py:37-41 -- logical code held by each slot of a 32-bit word
# in the "interleaved" layout.
INTERLEAVE = {
    4: (0, 2, 4, 6, 1, 3, 5, 7),
    2: (0, 4, 8, 12, 1, 5, 9, 13, 2, 6, 10, 14, 3, 7, 11, 15),
    8: (0, 2, 1, 3),
}


class Config:
    """Restates QuantConfig (dequant/packer.py:44-78)."""

    def __init__(self, bits=4, group_size=128, symmetric=True, layout="sequential"):
        if bits not in (2, 4, 8):
            raise ValueError(f"bits must be 2, 4 or 8, got {bits}")
        if layout not in ("sequential", "interleaved"):
            raise ValueError(f"unknown layout: {layout!r}")
        if group_size is not None and group_size <= 0:
            raise ValueError("group_size must be positive or None")
        self.bits, self.group_size, self.symmetric, self.layout = bits, group_size, symmetric, layout

    per_pack = property(lambda self: 32 // self.bits)
    qmax = property(lambda self: (1 << self.bits) - 1)
    bias = property(lambda self: 1 << (self.bits - 1))

    def effective_group_size(self, k):
        return k if self.group_size is None else self.group_size

    def order(self):
        """slot -> logical index (packer.py:153, :168)."""
        if self.layout == "interleaved":
            return INTERLEAVE[self.bits]
        return tuple(range(self.per_pack))


def quantize(w16, cfg):
    """fp16 [N, K] -> (codes int32 [N, K], scales fp16 [N, G], zeros fp16 | None).

    Follows dequant/packer.py:99-143 step by step, in fp32:
      symmetric : scale = amax / (2^(b-1) - 1), 0 -> 1, round to fp16,
                  q = round(w / scale) + 2^(b-1)                 (:113-127)
      asymmetric: scale = (max - min) / qmax, 0 -> 1, round to fp16,
                  zero = round(-min / scale) (unclamped),
                  q = round(w / scale) + zero                     (:128-137)
      both      : clamp to [0, qmax], int32                        (:139)
    round() is half-to-even (torch.round == np.rint).
    """
    w16 = np.asarray(w16)
    if w16.ndim != 2:
        raise ValueError(f"expected a 2-D weight, got shape {tuple(w16.shape)}")
    n, k = w16.shape
    gs = cfg.effective_group_size(k)
    if k % gs:
        raise ValueError(f"K={k} is not divisible by group_size={gs}")
    wf = w16.astype(np.float32).reshape(n, k // gs, gs)
    one = np.float32(1.0)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        if cfg.symmetric:
            amax = np.abs(wf).max(axis=-1, keepdims=True)
            scales = amax / np.float32(cfg.bias - 1)
            scales = np.where(scales == 0, one, scales).astype(np.float32)
            scales = scales.astype(np.float16).astype(np.float32)
            q = np.rint(wf / scales) + np.float32(cfg.bias)
            zeros = None
        else:
            wmax = wf.max(axis=-1, keepdims=True)
            wmin = wf.min(axis=-1, keepdims=True)
            scales = (wmax - wmin) / np.float32(cfg.qmax)
            scales = np.where(scales == 0, one, scales).astype(np.float32)
            scales = scales.astype(np.float16).astype(np.float32)
            zeros = np.rint(-wmin / scales)
            q = np.rint(wf / scales) + zeros
        q = np.clip(q, 0, cfg.qmax).astype(np.int32).reshape(n, k)
    scales16 = scales.reshape(n, -1).astype(np.float16)
    zeros16 = None if zeros is None else zeros.reshape(n, -1).astype(np.float16)
    return q, scales16, zeros16


def pack(q, cfg):
    """codes [N, K] -> int32 words [N, K/per] (dequant/packer.py:146-161).

    out |= (code[logical] & qmax) << (bits * slot) in int64, then the uint32
    bit pattern is kept in int32.
    """
    q = np.asarray(q)
    n, k = q.shape
    per = cfg.per_pack
    if k % per:
        raise ValueError(f"K={k} is not divisible by {per} values per word")
    blocks = q.reshape(n, k // per, per).astype(np.int64)
    out = np.zeros((n, k // per), dtype=np.int64)
    for slot, logical in enumerate(cfg.order()):
        out |= (blocks[:, :, logical] & cfg.qmax) << (cfg.bits * slot)
    return out.astype(np.uint32).view(np.int32)


def unpack(packed, cfg, k):
    """int32 words [N, K/per] -> codes int32 [N, K] (dequant/packer.py:164-174)."""
    packed = np.asarray(packed)
    n = packed.shape[0]
    per = cfg.per_pack
    words = packed.astype(np.int64) & 0xFFFFFFFF
    out = np.zeros((n, k // per, per), dtype=np.int32)
    for slot, logical in enumerate(cfg.order()):
        out[:, :, logical] = ((words >> (cfg.bits * slot)) & cfg.qmax).astype(np.int32)
    return out.reshape(n, k)


def _offsets(cfg, zeros16):
    if cfg.symmetric:
        return np.float32(cfg.bias)
    return zeros16.astype(np.float32)[..., None]


def dequantize(qweight, scales16, zeros16, cfg, shape):
    """fp16 [N, K] = fp16((code - offset) * scale) in fp32 (dequant/packer.py:177-189)."""
    n, k = shape
    gs = cfg.effective_group_size(k)
    q = unpack(qweight, cfg, k).reshape(n, k // gs, gs).astype(np.float32)
    s = scales16.astype(np.float32)[..., None]
    with np.errstate(invalid="ignore", over="ignore"):
        w = (q - _offsets(cfg, zeros16)) * s
    return w.reshape(n, k).astype(np.float16)


def exact_weight(qweight, scales16, zeros16, cfg, shape):
    """fp32 [N, K] = (code - offset) * scale WITHOUT the fp16 store.

    scripts/test_dequant_kernel.py:92-109 (same helper in
    scripts/test_quant_linear.py:92-105): the weight the fused kernel
    multiplies by, which isolates the dot product from packer.dequantize's
    own fp16 rounding.
    """
    n, k = shape
    gs = cfg.effective_group_size(k)
    q = unpack(qweight, cfg, k).reshape(n, k // gs, gs).astype(np.float32)
    s = scales16.astype(np.float32)[..., None]
    with np.errstate(invalid="ignore", over="ignore"):
        w = (q - _offsets(cfg, zeros16)) * s
    return w.reshape(n, k)


def gemv_reference(x16, w32):
    """(ref, absref) in float64: ref = x @ W^T, absref = |x| @ |W|^T.

    The reference's check is F.linear(x.float(), exact_weight) in fp32
    (scripts/test_dequant_kernel.py:131-132); float64 is used here so that the
    reference's own rounding does not eat into the tolerance.
    """
    x = np.asarray(x16).astype(np.float64)
    w = np.asarray(w32).astype(np.float64)
    return x @ w.T, np.abs(x) @ np.abs(w).T


def gemv_criterion(y16, ref, absref, depth=1):
    """|y - ref| <= depth * (2^-11 |ref| + 2^-20 |W|@|x|), elementwise.

    scripts/test_dequant_kernel.py:112-122 and scripts/test_quant_linear.py:85-89.
    Returns (ok, worst ratio err/tol).
    """
    y = np.asarray(y16).astype(np.float64)
    tol = depth * (2.0 ** -11 * np.abs(ref) + 2.0 ** -20 * absref)
    err = np.abs(y - ref)
    ratio = float((err / (tol + 1e-30)).max()) if err.size else 0.0
    return bool((err <= tol).all()), ratio


def rel_l2(y16, ref):
    """||y - ref||_2 / ||ref||_2 -- the north star's GEMV tolerance (<= 1e-3)."""
    y = np.asarray(y16).astype(np.float64)
    ref = np.asarray(ref).astype(np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(y - ref) / (den if den > 0 else 1.0))


def packed_nbytes(n, k, cfg):
    """PackedWeight.nbytes (dequant/packer.py:91-96)."""
    g = k // cfg.effective_group_size(k)
    nb = n * (k // cfg.per_pack) * 4 + n * g * 2
    if not cfg.symmetric:
        nb += n * g * 2
    return nb


def quantize_tensor(w16, cfg):
    """quantize + pack (dequant/packer.py:192-201). Returns (qweight, scales, zeros)."""
    q, s, z = quantize(w16, cfg)
    return pack(q, cfg), s, z
