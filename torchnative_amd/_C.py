"""The reference's `torch._C` entry points for this path, executed on the hip device.

Mirrors torchnative/rust/torch_c/src/quant.rs:107-418 (the block-quantised
tensor functions) and the device half of
`aten._scaled_dot_product_flash_attention_for_cpu` (aten.rs:10092-10440),
with the reference's names, argument meaning and error behaviour:
NotImplementedError for a refusal by name, RuntimeError in the reference's
wording for shape errors. A call with operands off the hip device refuses
instead of computing on the host.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np

from . import _lib
from ._lib import check, lib
from .tensor import Tensor, current_stream

QK4_0 = 32
Q4_0_TYPE_SIZE = 18
# format -> (elements per block, GGML bytes per block, device code bytes per block, C-ABI prefix)
_LAYOUT = {
    "q4_0": (32, 18, 16, "tn_q4_0"),
    "q8_0": (32, 34, 32, "tn_q8_0"),
    "q4_k": (256, 144, 144, "tn_q4_k"),  # one plane: the super-blocks, nibbles repacked (include/tnhip.h)
}
# dense formats (block size 1, candle k_quants.rs:2778-2910) -> (stored dtype, C ABI code, bytes per element)
_DENSE = {
    "f32": ("float32", _lib.TN_F32, 4),
    "f16": ("float16", _lib.TN_F16, 2),
    "bf16": ("bfloat16", _lib.TN_BF16, 2),
}
_FORMATS = tuple(_DENSE) + tuple(_LAYOUT)
_REFERENCE_FORMATS = ("f32", "f16", "bf16", "q4_0", "q4_1", "q5_0", "q5_1", "q8_0", "q8_1",
                      "q2_k", "q3_k", "q4_k", "q5_k", "q6_k", "q8_k")
SDPA_OP = "aten._scaled_dot_product_flash_attention_for_cpu.default"


def _block(fmt):
    """(elements per block, GGML bytes per block) of a format."""
    if fmt in _DENSE:
        return 1, _DENSE[fmt][2]
    return _LAYOUT[fmt][:2]


class QTensor:
    """A block-quantised weight [N, K] (the reference's `Repr::Quantized`,
    tensor.rs:970). On "hip" it is two device planes (the code bytes of every
    block and the f16 scales, include/tnhip.h), or for the dense formats
    f32/f16/bf16 one dense device tensor of that dtype; on "cpu" it is the
    GGML blob itself. The dtype tag is float32, as the reference's is
    (quant.rs:167)."""

    dtype = "float32"

    def __init__(self, shape, fmt, device, *, blob=None, qs=None, d=None):
        self.shape = tuple(int(s) for s in shape)
        self.format = fmt
        self.device = device
        self._blob = blob
        self._qs = qs
        self._d = d

    @property
    def n(self) -> int:
        return self.shape[0]

    @property
    def k(self) -> int:
        return self.shape[-1]

    @property
    def nblocks(self) -> int:
        return math.prod(self.shape) // _block(self.format)[0]

    @property
    def dense(self) -> bool:
        return self.format in _DENSE

    def _fn(self, op):
        return getattr(lib(), f"{_LAYOUT[self.format][3]}_{op}")

    def _planes(self):
        """The device plane pointers as the format's C functions take them."""
        return (self._qs.data_ptr(),) if self._d is None else (self._qs.data_ptr(), self._d.data_ptr())

    def __repr__(self):
        return f"QTensor(shape={self.shape}, format={self.format}, device={self.device})"


def _require_hip(op, *tensors):
    for t in tensors:
        if t is not None and getattr(t, "device", None) != "hip":
            raise NotImplementedError(
                f"{op}: operand on device {getattr(t, 'device', '?')!r}: this backend computes on the hip device "
                "only and does not fall back to the host; move the operands with .to('hip')"
            )


def _shape2(shape, fmt="q4_0"):
    if len(shape) != 2:
        raise NotImplementedError(f"{fmt} weights are 2-d [out_features, in_features] here, got shape {list(shape)}")
    return shape


def _planes(n, k, fmt):
    """Empty device planes for an [n, k] weight: (codes, f16 scales as bytes),
    or (super-blocks, None) for q4_k."""
    blk, _, code_bytes, _ = _LAYOUT[fmt]
    nb = n * k // blk
    codes = Tensor((nb * code_bytes,), "uint8", "hip")
    return codes, (None if fmt == "q4_k" else Tensor((nb * 2,), "uint8", "hip"))


def _quantized_formats():
    return list(_FORMATS)


def _format_check(op, fmt):
    if fmt not in _REFERENCE_FORMATS:
        raise ValueError(f"{op}: unknown quantisation format {fmt!r}; known: {', '.join(_REFERENCE_FORMATS)}")
    if fmt in ("q8_1", "q8_k"):
        raise NotImplementedError(
            f"{op}: {fmt} is an activation-side block format -- candle quantises the *input* to it inside "
            "vec_dot and no weight format names it as a VecDotType, so a weight stored this way has no matmul. "
            "Use q8_0."
        )
    if fmt not in _LAYOUT and fmt not in _DENSE:
        raise NotImplementedError(
            f"{op}: format {fmt!r} is not implemented on the hip device ({', '.join(_FORMATS)} are)")


def _quantize(t: Tensor, fmt: str) -> QTensor:
    """`_C._quantize(t, format)` (quant.rs:124-172): BlockQ4_0 / BlockQ8_0 /
    BlockQ4K::from_float on the device, or for f32/f16/bf16 the element-wise
    store (a copy, or half's round-to-nearest-even narrowing)."""
    op = "torch._C._quantize"
    _format_check(op, fmt)
    _require_hip(op, t)
    if t.dim() == 0:
        raise NotImplementedError(f"{op}: a 0-d tensor cannot be quantised")
    if t.dtype != "float32":
        raise NotImplementedError(f"{op}: the hip quantiser takes float32, got {t.dtype}")
    if fmt in _DENSE:
        n, k = _shape2(t.shape, fmt)
        stored, code, _ = _DENSE[fmt]
        w = Tensor((n, k), stored, "hip")
        check(lib().tn_dense_quantize(current_stream(), t.data_ptr(), n * k, code, w.data_ptr()))
        return QTensor((n, k), fmt, "hip", qs=w)
    blk = _LAYOUT[fmt][0]
    if t.shape[-1] % blk:
        raise NotImplementedError(
            f"{op}: {fmt} stores {blk} elements per block, so it must have their last dim divisible by block "
            f"size -- got {t.shape[-1]}, which is not a multiple of {blk} (shape {list(t.shape)})"
        )
    n, k = _shape2(t.shape, fmt)
    qs, d = _planes(n, k, fmt)
    q = QTensor((n, k), fmt, "hip", qs=qs, d=d)
    check(q._fn("quantize")(current_stream(), t.data_ptr(), n, k, *q._planes()))
    return q


def _quantized_from_blob(data: bytes, shape, fmt: str, device="cpu") -> QTensor:
    """`_C._quantized_from_blob(bytes, shape, format)` (quant.rs:230-262)."""
    op = "torch._C._quantized_from_blob"
    _format_check(op, fmt)
    blk, size = _block(fmt)
    numel = math.prod(shape)
    want = numel // blk * size
    if numel % blk or len(data) != want:
        raise ValueError(
            f"{op}: {fmt} stores {blk} elements in {size} bytes, so a {list(shape)} tensor needs "
            f"{want} bytes; got {len(data)}"
        )
    q = QTensor(_shape2(tuple(shape), fmt), fmt, "cpu", blob=bytes(data))
    return _quantized_to(q, device)


def _quantized_to(t: QTensor, device) -> QTensor:
    """`_C._quantized_to(t, device)` (quant.rs:384-405): the same blocks, byte
    for byte, on another device; same device returns the input itself."""
    dev = str(device)
    dev = "hip" if dev.startswith(("hip", "cuda")) else dev
    if dev not in ("cpu", "hip"):
        raise NotImplementedError(f"torch._C._quantized_to: device {device!r} is not implemented")
    if dev == t.device:
        return t
    n, k = t.shape
    if t.dense:
        if dev == "hip":
            w = Tensor((n, k), _DENSE[t.format][0], "hip")
            src = np.frombuffer(t._blob, dtype=np.uint8)
            check(lib().tn_memcpy_h2d(w.data_ptr(), src.ctypes.data, src.nbytes, current_stream()))
            return QTensor(t.shape, t.format, "hip", qs=w)
        return QTensor(t.shape, t.format, "cpu", blob=t._qs.bits().tobytes())
    if dev == "hip":
        blob = Tensor.from_numpy(np.frombuffer(t._blob, dtype=np.uint8), device="hip")
        qs, d = _planes(n, k, t.format)
        q = QTensor(t.shape, t.format, "hip", qs=qs, d=d)
        check(q._fn("from_blob")(current_stream(), blob.data_ptr(), n, k, *q._planes()))
        return q
    return QTensor(t.shape, t.format, "cpu", blob=_quantized_blob(t))


def _quantized_blob(t: QTensor) -> bytes:
    """`_C._quantized_blob(t)` (quant.rs:213-221): the raw GGML bytes."""
    if t.device == "cpu":
        return t._blob
    if t.dense:
        return t._qs.bits().tobytes()
    n, k = t.shape
    blob = Tensor((t.nblocks * _LAYOUT[t.format][1],), "uint8", "hip")
    check(t._fn("to_blob")(current_stream(), *t._planes(), n, k, blob.data_ptr()))
    return blob.bits().tobytes()


def _quantized_format(t: QTensor) -> str:
    return t.format


def _quantized_nbytes(t: QTensor) -> int:
    """What the weight costs (quant.rs:197-211): the GGML storage size."""
    return t.nblocks * _block(t.format)[1]


def _dequantize(t: QTensor) -> Tensor:
    """`_C._dequantize(t)` (quant.rs:180-189): dense float32, bit-exact."""
    op = "torch._C._dequantize"
    _require_hip(op, t)
    n, k = t.shape
    out = Tensor((n, k), "float32", "hip")
    if t.dense:
        check(lib().tn_dense_dequantize(current_stream(), t._qs.data_ptr(), _DENSE[t.format][1], n * k,
                                        out.data_ptr()))
        return out
    check(t._fn("dequantize")(current_stream(), *t._planes(), n, k, out.data_ptr()))
    return out


def _quantized_linear(input: Tensor, weight: QTensor, bias: Tensor | None = None, *, out_dtype=None) -> Tensor:
    """`_C._quantized_linear(input, weight, bias=None)` (quant.rs:286-369):
    input @ weight.T + bias with the reference's Q8_0 activation quantisation,
    bit-identical to its x86_64 arithmetic. float32 activations as the
    reference; bfloat16 activations are also taken on the hip device (widened
    exactly inside the quantising kernel)."""
    op = "torch._C._quantized_linear"
    if not isinstance(weight, QTensor):
        raise TypeError(f"{op}: weight must be a block-quantised tensor (torch._C._quantize), got {type(weight)}")
    if input.dtype not in ("float32", "bfloat16"):
        raise NotImplementedError(
            f"{op}: the activation must be float32, got torch.{input.dtype}. candle's QMatMul takes f32 or f16 "
            "only, and widening here would spend time the caller cannot see."
        )
    if input.device != weight.device:
        raise RuntimeError(
            f"{op}: Expected all tensors to be on the same device, but found at least two devices, "
            f"{input.device} (the input) and {weight.device} (the quantised weight). Move the module with "
            "`.to(device)`; QuantizedLinear moves its blocks byte for byte (torch._C._quantized_to)."
        )
    _require_hip(op, input, weight)
    out_features, in_features = weight.shape
    if input.dim() == 0 or input.shape[-1] != in_features:
        raise RuntimeError(
            f"{op}: mat1 and mat2 shapes cannot be multiplied ({list(input.shape)} and {in_features}x{out_features})"
        )
    if bias is not None:
        if bias.dtype != "float32":
            raise NotImplementedError(f"{op}: the bias must be float32, got torch.{bias.dtype}")
        if bias.shape != (out_features,):
            raise RuntimeError(f"{op}: bias shape {list(bias.shape)} does not match out_features {out_features}")
        _require_hip(op, bias)
    m = input.numel // in_features
    odt = out_dtype or "float32"
    if weight.dense:
        # QMatMul::from_arc widens f32/f16/bf16 up front and takes a plain
        # matmul (candle quantized/mod.rs:836-852): the dense linear itself
        if input.dtype != "float32" or odt != "float32":
            raise NotImplementedError(
                f"{op}: a {weight.format} weight is the dense control path, float32 in and out "
                f"(got torch.{input.dtype} in, torch.{odt} out)")
        out = Tensor(input.shape[:-1] + (out_features,), "float32", "hip")
        check(lib().tn_dense_linear(current_stream(), input.data_ptr(), m, in_features, weight._qs.data_ptr(),
                                    _DENSE[weight.format][1], out_features,
                                    bias.data_ptr() if bias is not None else None, out.data_ptr()))
        return out
    out = Tensor(input.shape[:-1] + (out_features,), odt, "hip")
    check(weight._fn("linear")(current_stream(), input.data_ptr(), _dt(input.dtype), m, in_features,
                               *weight._planes(), out_features,
                               bias.data_ptr() if bias is not None else None, out.data_ptr(), _dt(odt)))
    return out


def linear(input: Tensor, weight: Tensor, bias: Tensor | None = None) -> Tensor:
    """`F.linear(input, weight, bias)` for float32 operands on the hip device
    (bootstrap.py:13352-13357 -> aten.linear; the bias branch is addmm,
    aten.rs:9686-9700): input @ weight.T, each output one sequential fma chain
    over in_features (include/tnhip.h, tn_dense_linear), then + bias. The
    `_quantized_linear` of an f32 "quantised" weight is this same call."""
    op = "aten.linear.default"
    _require_hip(op, input, weight, bias)
    for name, t in (("input", input), ("weight", weight), ("bias", bias)):
        if t is not None and t.dtype != "float32":
            raise NotImplementedError(f"{op}: the hip linear takes float32, got torch.{t.dtype} for {name}")
    if weight.dim() != 2:
        raise RuntimeError(f"{op}: weight must be 2-d [out_features, in_features], got {list(weight.shape)}")
    out_features, in_features = weight.shape
    if input.dim() == 0 or input.shape[-1] != in_features:
        raise RuntimeError(
            f"{op}: mat1 and mat2 shapes cannot be multiplied ({list(input.shape)} and {in_features}x{out_features})")
    if bias is not None and bias.shape != (out_features,):
        raise RuntimeError(f"{op}: bias shape {list(bias.shape)} does not match out_features {out_features}")
    out = Tensor(input.shape[:-1] + (out_features,), "float32", "hip")
    check(lib().tn_dense_linear(current_stream(), input.data_ptr(), input.numel // in_features, in_features,
                                weight.data_ptr(), _lib.TN_F32, out_features,
                                bias.data_ptr() if bias is not None else None, out.data_ptr()))
    return out


def _dt(name):
    code = {"float32": _lib.TN_F32, "bfloat16": _lib.TN_BF16, "float16": _lib.TN_F16, "float64": _lib.TN_F64,
            "bool": _lib.TN_BOOL}.get(name)
    if code is None:
        raise NotImplementedError(f"dtype {name} has no C ABI code")
    return code


# --- SDPA -----------------------------------------------------------------------


def _scaled_dot_product_flash_attention(query: Tensor, key: Tensor, value: Tensor, dropout_p: float = 0.0,
                                        is_causal: bool = False, *, attn_mask: Tensor | None = None,
                                        scale: float | None = None, _check_only: bool = False):
    """The device half of aten._scaled_dot_product_flash_attention_for_cpu
    (aten.rs:10092-10440). Returns (out, logsumexp); out is row-major
    [B,Hq,L,D] in the query dtype, logsumexp float32 [B,Hq,L]."""
    op = SDPA_OP
    if not (query.dtype == key.dtype == value.dtype):
        raise RuntimeError(f"{op}: Expected query, key, and value to have the same dtype, but got query.dtype: "
                           f"{query.dtype} key.dtype: {key.dtype} and value.dtype: {value.dtype} instead.")
    if query.dtype not in ("float32", "float64", "bfloat16", "float16"):
        raise RuntimeError("scaled_dot_product_attention_flash_attention: Expected data type in FP32, FP64, BF16, "
                           f"FP16, but got {query.dtype} instead.")
    if dropout_p > 0.0:
        raise RuntimeError("scaled_dot_product_attention_flash_attention: Currently do not support dropout > 0")
    for t in (query, key, value):
        if t.dim() != 4:
            raise RuntimeError("scaled_dot_product_attention_flash_attention: Accept only 4 dims inputs shape of "
                               "{B, H, T, K}")
    if attn_mask is not None and attn_mask.dtype not in (query.dtype, "float32"):
        raise RuntimeError("scaled_dot_product_attention_flash_attention: Attention mask is the same data type as "
                           "query")
    if attn_mask is not None and query.dtype == "float64" and attn_mask.dtype == "float32":
        raise NotImplementedError(
            "aten._scaled_dot_product_flash_attention_for_cpu: a float32 attn_mask on a float64 query is refused. "
            "Pass the mask as float64.")
    _require_hip(op, query, key, value, attn_mask)
    B, Hq, L, D = query.shape
    Bk, Hkv, S, Dk = key.shape
    for name, t in (("key", key), ("value", value)):
        if t.shape[0] != B or t.shape[2] != S or t.shape[3] != D or t.shape[1] != Hkv:
            raise RuntimeError(f"{op}: query {list(query.shape)} and {name} {list(t.shape)} do not describe one "
                               "attention -- batch, key length and head dimension all have to agree")
    if _check_only:
        return None
    return _sdpa_call(query, key, value, is_causal, attn_mask, scale)


def _mask_strides(op, mask: Tensor, B, Hq, L, S):
    """Element strides of `mask` (dense in its own shape) broadcast onto
    [B, Hq, L, S]: numpy's rule, a missing or size-1 dim repeats (stride 0).
    The reference broadcasts the mask onto the scores the same way
    (aten.rs:10293-10303); here the kernels read it where it lies."""
    shape = tuple(mask.shape)
    if len(shape) > 4 or any(s not in (1, t) for s, t in zip(shape[::-1], (S, L, Hq, B))):
        raise RuntimeError(f"{op}: attn_mask of shape {list(shape)} cannot be broadcast to [{B}, {Hq}, {L}, {S}]")
    full = (1,) * (4 - len(shape)) + shape
    strides, acc = [0] * 4, 1
    for i in range(3, -1, -1):
        strides[i] = 0 if full[i] == 1 else acc
        acc *= full[i]
    return (ctypes.c_int64 * 4)(*strides)


def _sdpa_call(query, key, value, is_causal, attn_mask, scale):
    B, Hq, L, D = query.shape
    Hkv, S = key.shape[1], key.shape[2]
    strides = _mask_strides(SDPA_OP, attn_mask, B, Hq, L, S) if attn_mask is not None else None
    out = Tensor((B, Hq, L, D), query.dtype, "hip")
    lse = Tensor((B, Hq, L), "float64" if query.dtype == "float64" else "float32", "hip")
    sc = float("nan") if scale is None else float(scale)
    check(lib().tn_sdpa_fwd(current_stream(), _dt(query.dtype), query.data_ptr(), key.data_ptr(), value.data_ptr(),
                            B, Hq, Hkv, L, S, D, attn_mask.data_ptr() if attn_mask is not None else None,
                            _dt(attn_mask.dtype) if attn_mask is not None else 0, strides, int(bool(is_causal)), sc,
                            out.data_ptr(), lse.data_ptr()))
    return out, lse


def scaled_dot_product_attention(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False, scale=None,
                                 enable_gqa=False):
    """`F.scaled_dot_product_attention` as the reference's CIA body reaches the
    flash op (bootstrap.py:13036-13080): returns the output only. A bool mask
    is taken as the additive where(mask, 0, -inf) in the query's dtype that
    the CIA body builds before the flash call (bootstrap.py:12918-12925,
    :13065-13066); the kernels read the bool bytes in place (TN_BOOL), so no
    converted copy is made."""
    if query.dim() == 4 and key.dim() == 4 and query.shape[1] != key.shape[1] and not enable_gqa:
        raise RuntimeError("scaled_dot_product_attention: query and key head counts differ; pass enable_gqa=True")
    if attn_mask is not None and is_causal:
        raise RuntimeError("_scaled_dot_product_attention: Explicit attn_mask should not be set when is_causal=True")
    if attn_mask is None or attn_mask.dtype != "bool":
        out, _ = _scaled_dot_product_flash_attention(query, key, value, dropout_p, is_causal, attn_mask=attn_mask,
                                                     scale=scale)
        return out
    # the flash op's own checks, with the mask as the query-dtype tensor it stands for
    _scaled_dot_product_flash_attention(query, key, value, dropout_p, is_causal, attn_mask=None, scale=scale,
                                        _check_only=True)
    _require_hip(SDPA_OP, attn_mask)
    out, _ = _sdpa_call(query, key, value, is_causal, attn_mask, scale)
    return out


def sdpa_decode(query: Tensor, k_cache: Tensor, v_cache: Tensor, lens: Tensor, max_len: int,
                scale: float | None = None):
    """One query token per sequence over per-sequence KV caches
    [B, Hkv, cap, D] (kernels/kv_cache.py:92-114's layout), sequence b using
    keys 0..lens[b]-1. query [B, Hq, D] (or [B, Hq, 1, D]). Returns (out, lse)."""
    op = "sdpa_decode"
    _require_hip(op, query, k_cache, v_cache, lens)
    if lens.dtype != "int32":
        raise NotImplementedError(f"{op}: lens must be int32, got {lens.dtype}")
    q = query.view(query.shape[0], query.shape[1], query.shape[-1]) if query.dim() == 4 else query
    B, Hq, D = q.shape
    Bk, Hkv, cap, Dk = k_cache.shape
    if Bk != B or Dk != D or v_cache.shape != k_cache.shape or lens.shape != (B,):
        raise RuntimeError(f"{op}: query {list(q.shape)}, caches {list(k_cache.shape)}/{list(v_cache.shape)} and "
                           f"lens {list(lens.shape)} do not describe one decode step")
    if not (q.dtype == k_cache.dtype == v_cache.dtype):
        raise RuntimeError(f"{op}: query and caches must share a dtype")
    out = Tensor(query.shape, q.dtype, "hip")
    lse = Tensor((B, Hq), "float32", "hip")
    sc = float("nan") if scale is None else float(scale)
    check(lib().tn_sdpa_decode(current_stream(), _dt(q.dtype), q.data_ptr(), k_cache.data_ptr(),
                               v_cache.data_ptr(), B, Hq, Hkv, cap, D, lens.data_ptr(), int(max_len), sc,
                               out.data_ptr(), lse.data_ptr()))
    return out, lse


_DISPATCH = {SDPA_OP: _scaled_dot_product_flash_attention}


def _aten_dispatch(op: str, *args, **kwargs):
    """The whitelist door (vulkan.rs:1100-1223 shape): ops this backend
    executes run; anything else refuses, naming the op and the list."""
    fn = _DISPATCH.get(op)
    if fn is None:
        raise NotImplementedError(
            f"{op} is not implemented for the hip device; it executes: {', '.join(sorted(_DISPATCH))}")
    return fn(*args, **kwargs)


# --- probe / counters (device.rs:1671-1708, vulkan.rs:2138-2268 shape) ---------


def _hip_probe() -> dict:
    buf = ctypes.create_string_buffer(512)
    check(lib().tn_probe(buf, 512))
    out = {}
    for part in buf.value.decode().split(";"):
        k, _, v = part.partition("=")
        out[k] = int(v) if v.isdigit() else v
    return out


def _hip_counters() -> dict:
    c = _lib.Counters()
    check(lib().tn_counters(ctypes.byref(c)))
    return {f: int(getattr(c, f)) for f, _ in _lib.Counters._fields_}


def _hip_counters_reset() -> None:
    check(lib().tn_counters_reset())


def _hip_ops() -> list:
    return lib().tn_ops().decode().split(",")
