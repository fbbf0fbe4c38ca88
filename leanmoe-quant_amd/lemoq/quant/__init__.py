"""Weight formats and quantisation (reference: ``src/lemoq/quant``): per-group RTN
at 4 / 8 bits on the device (``rtn``), 4-bit packing and byte costs (``pack``),
MXFP4 (``mxfp4``), the format ids of the dequant kernels (``formats``),
``QuantLinear`` and the model-level helpers (``linear``), and the stable entry
points re-exported here (``api``)."""

from __future__ import annotations

from lemoq.quant.api import REMEDIATION_LADDER, QuantizedLinear, dequantize_reference, quantize_linear

__all__ = ["REMEDIATION_LADDER", "QuantizedLinear", "dequantize_reference", "quantize_linear"]
