"""`QuantizedLinear` and `quantize_` for the hip device.

The reference's caller of the quantised linear
(torchnative/python/torchnative/quant/__init__.py:100-365): every dense
linear of a model is swapped for a layer whose weight is a block-quantised
tensor, lm_head included unless a predicate says otherwise (:300-312); the
bias stays dense float32; the blocks move byte for byte when the model moves
(`_apply`, :221-237, through `_quantized_to`, never re-quantised); and the
call returns a report of what was replaced, what was skipped and why, and
the bytes on both sides (:255-297). A layer the format cannot hold (in
features not a multiple of the block size) is skipped with the quantiser's
refusal as its reason, never silently left dense. Models here are
`torchnative_amd.nn` trees.
"""

from __future__ import annotations

from . import _C
from .nn import Linear
from .tensor import Tensor


class QuantizedLinear:
    """A linear layer over a block-quantised weight [out_features, in_features]
    (q4_0, q8_0 or q4_k, or the dense control formats f32/f16/bf16): forward
    is `_quantized_linear(x, qweight, bias)`."""

    def __init__(self, qweight: "_C.QTensor", bias: Tensor | None = None):
        self.qweight = qweight
        self.bias = bias
        self.format = qweight.format
        self.out_features, self.in_features = qweight.shape

    @classmethod
    def from_linear(cls, mod, format: str = "q4_0") -> "QuantizedLinear":
        """Quantise a dense layer's weight with `_quantize` on the device (a
        host weight is uploaded first). Raises NotImplementedError, naming why,
        when the format cannot hold the weight."""
        w = mod.weight if mod.weight.device == "hip" else mod.weight.to("hip")
        bias = mod.bias
        if bias is not None and bias.device != "hip":
            bias = bias.to("hip")
        return cls(_C._quantize(w, format), bias)

    @classmethod
    def from_dense(cls, weight: Tensor, bias: Tensor | None = None, format: str = "q4_0") -> "QuantizedLinear":
        return cls.from_linear(Linear(weight, bias), format)

    @classmethod
    def from_blob(cls, blob: bytes, out_features: int, in_features: int, bias: Tensor | None = None,
                  device="hip", format: str = "q4_0") -> "QuantizedLinear":
        """A layer over existing GGML blocks (a GGUF file's own)."""
        return cls(_C._quantized_from_blob(blob, (out_features, in_features), format, device), bias)

    def _apply(self, device):
        """Move the blocks byte for byte (`_quantized_to`) and the bias."""
        self.qweight = _C._quantized_to(self.qweight, device)
        if self.bias is not None:
            self.bias = self.bias.to(device)
        return self

    to = _apply

    @property
    def device(self) -> str:
        return self.qweight.device

    def forward(self, x: Tensor, out_dtype=None) -> Tensor:
        return _C._quantized_linear(x, self.qweight, self.bias, out_dtype=out_dtype)

    __call__ = forward

    def __repr__(self):
        return (f"QuantizedLinear(in_features={self.in_features}, out_features={self.out_features}, "
                f"format={self.format}, bias={self.bias is not None}, device={self.device})")


class QuantizeReport:
    """What `quantize_` did: the layers replaced, the layers skipped with the
    reason for each, and the weight bytes before and after for the replaced
    layers only (everything else in the model is unchanged)."""

    def __init__(self, format: str):
        self.format = format
        self.replaced: list = []
        self.skipped: list = []  # (name, reason)
        self.dense_bytes = 0
        self.quantized_bytes = 0

    @property
    def ratio(self) -> float:
        return self.dense_bytes / self.quantized_bytes if self.quantized_bytes else float("nan")

    def reasons(self) -> dict:
        """reason -> the layers skipped for it, in model order."""
        out: dict = {}
        for name, why in self.skipped:
            out.setdefault(why, []).append(name)
        return out

    def __str__(self):
        head = (f"quantize_ to {self.format}: {len(self.replaced)} layers replaced, {len(self.skipped)} skipped; "
                f"the replaced weights went from {self.dense_bytes} to {self.quantized_bytes} bytes "
                f"({self.ratio:.2f}x smaller; other parameters unchanged)")
        lines = [head]
        for why, names in self.reasons().items():
            lines.append(f"  {len(names)} skipped because {why}: {', '.join(names)}")
        return "\n".join(lines)


def _why(exc: Exception) -> str:
    """The part of a quantiser refusal that tells layers apart: the clause
    after the op name."""
    text = str(exc)
    return text.split(": ", 1)[1] if text.startswith("torch._C.") and ": " in text else text


def quantize_(model, format: str = "q8_0", predicate=None) -> QuantizeReport:
    """Replace every `Linear` under `model` with a `QuantizedLinear`, in place,
    and return the report. `predicate(name, module) -> bool` narrows the
    choice; lm_head is not treated specially (the reference leaves that
    choice to the predicate, quant/__init__.py:300-312). A layer whose
    weight the format cannot hold stays dense and is reported with the
    quantiser's reason. Handing over a bare Linear, or a model with no
    Linear in it, raises ValueError: nothing would be replaced, and an empty
    report would read as success."""
    report = QuantizeReport(format)
    if isinstance(model, Linear):
        raise ValueError("quantize_ rebinds the children of the module it is given, so a bare Linear cannot be "
                         "replaced this way; build one with QuantizedLinear.from_linear(layer, format) and assign "
                         "it, or pass the model that holds the layer")
    todo = []
    for name, parent in model.named_modules():
        if not hasattr(parent, "named_children"):
            continue
        for child_name, child in parent.named_children():
            if not isinstance(child, Linear):
                continue
            full = f"{name}.{child_name}" if name else child_name
            if predicate is not None and not predicate(full, child):
                report.skipped.append((full, "excluded by the predicate"))
            else:
                todo.append((parent, child_name, full, child))
    for parent, child_name, full, child in todo:
        try:
            q = QuantizedLinear.from_linear(child, format)
        except NotImplementedError as e:
            report.skipped.append((full, _why(e)))
            continue
        setattr(parent, child_name, q)
        report.replaced.append(full)
        report.dense_bytes += child.weight.numel * 4
        report.quantized_bytes += _C._quantized_nbytes(q.qweight)
    if not report.replaced and not report.skipped:
        raise ValueError(f"quantize_: {type(model).__name__} holds no Linear layer, so nothing was quantised")
    return report
