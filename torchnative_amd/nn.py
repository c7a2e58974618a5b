"""The few module-tree pieces the quantisation swap needs.

`quantize_` (quant.py) walks a model the way the reference walks an
`nn.Module` (torchnative/python/torchnative/quant/__init__.py:300-365):
parents list their children by name, a child is rebound with `setattr`, and
`.to(device)` visits every module so that each moves what it owns. These
classes give that shape over this package's tensors: `Module` records child
modules in assignment order, `Linear` holds a float32 weight [out, in] and
an optional bias (its forward is the dense F.linear), and `ModuleList`
numbers its children.
"""

from __future__ import annotations

import numpy as np

from .tensor import Tensor

__all__ = ["Module", "Linear", "ModuleList"]


class Module:
    """A node of a model: attributes that are Modules are its children."""

    def __init__(self):
        object.__setattr__(self, "_children", {})

    def __setattr__(self, name, value):
        kids = self.__dict__.get("_children")
        if kids is None:
            raise AttributeError(f"{type(self).__name__}.__init__ must call Module.__init__ first")
        if isinstance(value, Module) or _is_module_like(value):
            kids[name] = value
        else:
            kids.pop(name, None)
        object.__setattr__(self, name, value)

    def named_children(self):
        return list(self._children.items())

    def named_modules(self, prefix: str = ""):
        """This module and every descendant, depth first, with dotted names."""
        out = [(prefix, self)]
        for name, child in self._children.items():
            full = f"{prefix}.{name}" if prefix else name
            if isinstance(child, Module):
                out.extend(child.named_modules(full))
            else:
                out.append((full, child))
        return out

    def _apply(self, device):
        """Move what this module owns (subclasses override), then its children."""
        for child in self._children.values():
            child._apply(device)
        return self

    def to(self, device):
        return self._apply(device)


def _is_module_like(v) -> bool:
    # a QuantizedLinear (quant.py) is a leaf module without deriving from Module
    return hasattr(v, "_apply") and hasattr(v, "forward") and not isinstance(v, Tensor)


class ModuleList(Module):
    def __init__(self, modules=()):
        super().__init__()
        for i, m in enumerate(modules):
            setattr(self, str(i), m)

    def __getitem__(self, i):
        return getattr(self, str(i))

    def __len__(self):
        return len(self._children)


class Linear(Module):
    """A dense linear layer: y = x W^T + b, W float32 [out_features, in_features].
    forward is `F.linear` on the hip device (_C.linear), the dense side of the
    `format="f32"` exactness control."""

    def __init__(self, weight, bias=None, device="hip"):
        super().__init__()
        w = weight if isinstance(weight, Tensor) else Tensor.from_numpy(np.asarray(weight, np.float32),
                                                                       device=device)
        if w.dim() != 2 or w.dtype != "float32":
            raise ValueError(f"Linear: the weight is float32 [out_features, in_features], got {w.dtype} "
                             f"{list(w.shape)}")
        b = None
        if bias is not None:
            b = bias if isinstance(bias, Tensor) else Tensor.from_numpy(np.asarray(bias, np.float32), device=device)
        self.weight, self.bias = w, b
        self.out_features, self.in_features = w.shape

    def _apply(self, device):
        self.weight = self.weight.to(device)
        if self.bias is not None:
            self.bias = self.bias.to(device)
        return self

    def forward(self, x):
        from . import _C

        return _C.linear(x, self.weight, self.bias)

    __call__ = forward
