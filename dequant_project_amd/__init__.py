"""MI355X (gfx950) fused dequant + GEMV engine for packed INT2/INT4/INT8 weights.

Drop-in for the decode path of KrishnaI2424/Dequant_Project:

  packer         the packed-weight format and offline quantizer (same bytes)
  quant_linear   QuantLinear / gemv / dequantize_cuda / quantize_model
  byte_model     analytical bytes per call / per decode step, MI355X roofline
  dequant_cuda   the native extension (gemv / dequantize / unpack / add_one),
                 a thin torch layer over the C ABI of include/dequant_hip.h

Native code is built in-tree with `python -m dequant_project_amd.build`.
"""

from .packer import (PackedWeight, QuantConfig, dequantize, pack, quantize,  # noqa: F401
                     quantize_tensor, unpack)
from .quant_linear import (MAX_M, PROJ, QuantLinear, dequantize_cuda, gemv, gemv_grouped,  # noqa: F401
                           quantize_model)

__version__ = "0.1.0"
