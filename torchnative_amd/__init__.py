"""torchnative_amd: MI355X (gfx950) HIP backend for torchnative's
quantised-inference hot path -- the q4_0 weight-only linear and
scaled_dot_product_attention -- behind a C ABI (include/tnhip.h,
libtnhip.so) and a Python mirror of the reference's `torch._C` entry points.
"""

from . import _C, device, gguf, nn, quant, tensor
from ._C import (
    QTensor,
    _aten_dispatch,
    _dequantize,
    _hip_counters,
    _hip_ops,
    _hip_probe,
    _quantize,
    _quantized_blob,
    _quantized_format,
    _quantized_formats,
    _quantized_from_blob,
    _quantized_linear,
    _quantized_nbytes,
    _quantized_to,
    scaled_dot_product_attention,
    sdpa_decode,
)
from .quant import QuantizedLinear, QuantizeReport, quantize_
from .tensor import Event, Stream, Tensor, empty, synchronize, tensor, zeros

__all__ = [
    "QTensor", "QuantizedLinear", "QuantizeReport", "quantize_", "Tensor", "Stream", "Event", "empty", "zeros", "tensor",
    "synchronize", "_quantize", "_dequantize", "_quantized_linear", "_quantized_to", "_quantized_blob",
    "_quantized_from_blob", "_quantized_format", "_quantized_formats", "_quantized_nbytes", "_aten_dispatch",
    "scaled_dot_product_attention", "sdpa_decode", "_hip_probe", "_hip_counters", "_hip_ops",
]
