"""The reference's CPU torch path, restated -- TEST / BASELINE INFRASTRUCTURE ONLY.

Used by bench.py's cpu_baseline leg (timed on the host cores of the GPU box)
and by tests as a third, torch-based restatement. It follows the path the
reference's Python takes when the weight is materialized:

  unpack      dequant/packer.py:164-174   int64 shifts and masks per slot
  dequantize  dequant/packer.py:177-189   fp16((q - offset) * scale), fp32 math
  linear      F.linear(x.float(), W.float())  (the reference's fp32 check,
              scripts/test_dequant_kernel.py:131-132; the module's M > 8 path
              dequant/quant_linear.py:131-132 is F.linear over the fp16 W)

Parity pinning: tests/test_oracle_cpu_path.py checks unpack / dequantize
against the golden vectors and the GEMV against oracle.packer_ref.
"""

import torch
import torch.nn.functional as F

INTERLEAVE = {
    4: [0, 2, 4, 6, 1, 3, 5, 7],
    2: [0, 4, 8, 12, 1, 5, 9, 13, 2, 6, 10, 14, 3, 7, 11, 15],
    8: [0, 2, 1, 3],
}


def unpack(qweight, bits, interleaved, k):
    """int32 words [N, K*bits/32] -> int32 codes [N, K] (logical order)."""
    per = 32 // bits
    qmax = (1 << bits) - 1
    order = INTERLEAVE[bits] if interleaved else range(per)
    words = qweight.to(torch.int64) & 0xFFFFFFFF
    out = torch.empty(qweight.shape[0], k // per, per, dtype=torch.int32)
    for slot, logical in enumerate(order):
        out[:, :, logical] = ((words >> (bits * slot)) & qmax).to(torch.int32)
    return out.reshape(qweight.shape[0], k)


def dequantize(qweight, scales, zeros, bits, group_size, symmetric, interleaved, k):
    """fp16 [N, K] = fp16((code - offset) * scale) computed in fp32."""
    n = qweight.shape[0]
    q = unpack(qweight, bits, interleaved, k).reshape(n, k // group_size, group_size).float()
    off = float(1 << (bits - 1)) if symmetric else zeros.float().unsqueeze(-1)
    return ((q - off) * scales.float().unsqueeze(-1)).reshape(n, k).to(torch.float16)


def gemv(x, qweight, scales, zeros, bits, group_size, symmetric, interleaved):
    """y = F.linear(x.float(), dequantize(...).float()) -> fp32 [M, N]."""
    k = x.shape[-1]
    w = dequantize(qweight, scales, zeros, bits, group_size, symmetric, interleaved, k)
    return F.linear(x.float(), w.float())
