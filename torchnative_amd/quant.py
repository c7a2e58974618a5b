"""`QuantizedLinear` and `quantize_` for the hip device.

Mirrors torchnative/python/torchnative/quant/__init__.py:100-365: a linear
layer whose weight is a block-quantised tensor held as a plain attribute, whose
forward is `_quantized_linear(x, qweight, bias)`, whose bias stays dense
float32, and whose blocks move byte for byte on `.to()` (`_quantized_to`,
never re-quantised).
"""

from __future__ import annotations

from . import _C
from .tensor import Tensor


class QuantizedLinear:
    """nn.Linear with a block-quantised (q4_0 or q8_0) weight [out_features, in_features]."""

    def __init__(self, qweight: "_C.QTensor", bias: Tensor | None = None):
        self.qweight = qweight
        self.bias = bias
        self.out_features, self.in_features = qweight.shape

    @classmethod
    def from_dense(cls, weight: Tensor, bias: Tensor | None = None, format: str = "q4_0") -> "QuantizedLinear":
        """`QuantizedLinear.from_linear` (quant/__init__.py:141-152): quantise a
        dense float32 weight with `_quantize` (on its device)."""
        return cls(_C._quantize(weight, format), bias)

    @classmethod
    def from_blob(cls, blob: bytes, out_features: int, in_features: int, bias: Tensor | None = None,
                  device="hip", format: str = "q4_0") -> "QuantizedLinear":
        """A layer over an existing GGML blob (a GGUF file's own blocks)."""
        return cls(_C._quantized_from_blob(blob, (out_features, in_features), format, device), bias)

    def to(self, device) -> "QuantizedLinear":
        """quant/__init__.py:221-237: blocks move byte for byte."""
        self.qweight = _C._quantized_to(self.qweight, device)
        if self.bias is not None:
            self.bias = self.bias.to(device)
        return self

    def forward(self, x: Tensor, out_dtype=None) -> Tensor:
        return _C._quantized_linear(x, self.qweight, self.bias, out_dtype=out_dtype)

    __call__ = forward

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"format={_C._quantized_format(self.qweight)}, bias={self.bias is not None}")


def quantize_(layers: dict, format: str = "q4_0", predicate=None) -> dict:
    """Swap every dense linear in ``layers`` (name -> (weight, bias)) for a
    QuantizedLinear, lm_head included unless ``predicate(name)`` says no
    (quant/__init__.py:300-365). Layers whose in_features is not a multiple of
    the block size are left dense and reported, as the reference groups its
    skips by the refusal message."""
    out, skipped = {}, {}
    for name, (w, b) in layers.items():
        if predicate is not None and not predicate(name):
            out[name] = (w, b)
            continue
        try:
            out[name] = QuantizedLinear.from_dense(w, b, format)
        except NotImplementedError as e:
            skipped[name] = str(e)
            out[name] = (w, b)
    out["__skipped__"] = skipped
    return out
