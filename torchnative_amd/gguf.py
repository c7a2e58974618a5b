"""GGUF checkpoints for the hip device.

What the reference does with a GGUF file (torchnative/python/torchnative/gguf,
`load_tensor` at __init__.py:135-170 and `quantized_linear` at :173-201) is:
read the container, hand dense tensors over in their own dtype, and hand
block tensors over as their GGML blocks, never decoded on the way in. This
module does the same for the hip device: a block tensor's bytes go to
`_quantized_from_blob`, which splits them into the device's code and scale
planes (tn_q4_0_from_blob, tn_q8_0_from_blob, tn_q4_k_from_blob), so
`_quantized_blob` of a loaded weight gives back the file's bytes.

The container, as the GGUF specification lays it out (v2 and v3, little
endian): a 24-byte header (b"GGUF", u32 version, u64 tensor count, u64
metadata count); the metadata pairs (string key, u32 value type, value); the
tensor descriptors (string name, u32 dimension count, u64 extents fastest
first, u32 GGML type, u64 offset into the data section); zero padding to
`general.alignment` (32 when absent); the data section. A string is a u64
byte count and the bytes; an array is a u32 element type, a u64 count and
the elements.

The file is memory-mapped; `scan` walks it once, checking every read against
the file's size, and everything after that is a slice of the map.
"""

from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass
from typing import NamedTuple, Optional

import numpy as np

__all__ = ["GGUFFile", "GGUFTensorInfo", "TensorEntry", "GGMLType", "GGML_TYPES", "GGUFFormatError",
           "UnsupportedGGUF", "type_name", "refusal", "load_tensor", "quantized_linear"]


class GGUFFormatError(ValueError):
    """The bytes break the GGUF layout."""


class UnsupportedGGUF(NotImplementedError):
    """Valid GGUF that this backend does not load; the message says why."""


class GGMLType(NamedTuple):
    """One row of the GGML type table. `load` is "dense" (read as `what`, a
    dtype), "blocks" (kept as the quantised format `what`) or "no" (refused;
    `what` keys the reason)."""

    id: int
    name: str
    block: Optional[int]  # elements per block
    size: Optional[int]  # bytes per block
    load: str
    what: str


# The GGML type ids with their elements and bytes per block are the file
# format's own (ggml's type traits); a reader has to agree with them exactly.
GGML_TYPES = {t.id: t for t in (GGMLType(*row) for row in (
    (0, "F32", 1, 4, "dense", "float32"),
    (1, "F16", 1, 2, "dense", "float16"),
    (2, "Q4_0", 32, 18, "blocks", "q4_0"),
    (3, "Q4_1", 32, 20, "no", "other_blocks"),
    (6, "Q5_0", 32, 22, "no", "other_blocks"),
    (7, "Q5_1", 32, 24, "no", "other_blocks"),
    (8, "Q8_0", 32, 34, "blocks", "q8_0"),
    (9, "Q8_1", 32, 36, "no", "rhs_only"),
    (10, "Q2_K", 256, 84, "no", "other_blocks"),
    (11, "Q3_K", 256, 110, "no", "other_blocks"),
    (12, "Q4_K", 256, 144, "blocks", "q4_k"),
    (13, "Q5_K", 256, 176, "no", "other_blocks"),
    (14, "Q6_K", 256, 210, "no", "other_blocks"),
    (15, "Q8_K", 256, 292, "no", "rhs_only"),
    (16, "IQ2_XXS", 256, 66, "no", "iq"),
    (17, "IQ2_XS", 256, 74, "no", "iq"),
    (18, "IQ3_XXS", 256, 98, "no", "iq"),
    (19, "IQ1_S", 256, 50, "no", "iq"),
    (20, "IQ4_NL", 32, 18, "no", "iq"),
    (21, "IQ3_S", 256, 110, "no", "iq"),
    (22, "IQ2_S", 256, 82, "no", "iq"),
    (23, "IQ4_XS", 256, 136, "no", "iq"),
    (24, "I8", 1, 1, "no", "integer"),
    (25, "I16", 1, 2, "no", "integer"),
    (26, "I32", 1, 4, "no", "integer"),
    (27, "I64", 1, 8, "no", "integer"),
    (28, "F64", 1, 8, "no", "integer"),
    (29, "IQ1_M", 256, 56, "no", "iq"),
    (30, "BF16", 1, 2, "dense", "bfloat16"),
    (31, "Q4_0_4_4", None, None, "no", "retired"),
    (32, "Q4_0_4_8", None, None, "no", "retired"),
    (33, "Q4_0_8_8", None, None, "no", "retired"),
    (34, "TQ1_0", 256, 54, "no", "iq"),
    (35, "TQ2_0", 256, 66, "no", "iq"),
    (36, "IQ4_NL_4_4", None, None, "no", "retired"),
    (37, "IQ4_NL_4_8", None, None, "no", "retired"),
    (38, "IQ4_NL_8_8", None, None, "no", "retired"),
    (39, "MXFP4", 32, 17, "no", "iq"),
))}

# Why a type is not loaded on this backend.
_WHY_NOT = {
    "other_blocks": "is a block format with no hip kernel here; the hip device runs q4_0, q8_0 and q4_k "
                    "blocks, so re-quantise the model to one of those",
    "rhs_only": "only ever exists as the quantised activation inside a block dot product, so no weight is "
                "stored in it",
    "iq": "has no storage type in the reference's candle either; re-quantise the model to q4_0, q8_0 or q4_k",
    "integer": "is a plain numeric element type that checkpoints do not use for weights; it is not loaded",
    "retired": "is an interleaved layout that ggml no longer writes; its files have to be re-converted",
}


def type_name(ggml_type: int) -> str:
    t = GGML_TYPES.get(ggml_type)
    return t.name if t else f"unknown#{ggml_type}"


def refusal(ggml_type: int, tensor_name: str | None = None):
    """The UnsupportedGGUF a tensor of this type would raise, or None if it loads."""
    subject = f"tensor {tensor_name!r}" if tensor_name is not None else "a tensor"
    t = GGML_TYPES.get(ggml_type)
    if t is None:
        return UnsupportedGGUF(f"{subject} has GGML type id {ggml_type}, which is not in this reader's table; "
                               "nothing is guessed about its layout")
    if t.load == "no":
        return UnsupportedGGUF(f"{subject} is {t.name}, which {_WHY_NOT[t.what]}")
    return None


@dataclass(frozen=True)
class TensorEntry:
    """One tensor descriptor. `ne` is GGUF's order (fastest first); `shape`
    is torch's (reversed), so a linear weight with ne = [in, out] has shape
    (out, in). `offset` is absolute in the file. `nbytes` is None when the
    type's size is not known (the tensor is listed but never read)."""

    name: str
    ggml_type: int
    ne: tuple
    offset: int
    nbytes: Optional[int]

    @property
    def shape(self) -> tuple:
        return tuple(reversed(self.ne))

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.ne:
            n *= d
        return n

    @property
    def type_name(self) -> str:
        return type_name(self.ggml_type)

    @property
    def kind(self) -> str:
        """"dense", "block" or "refused"."""
        t = GGML_TYPES.get(self.ggml_type)
        return {"dense": "dense", "blocks": "block"}.get(t.load, "refused") if t else "refused"

    @property
    def format(self):
        """The quantised format a block tensor loads as (`_quantized_formats()`), else None."""
        t = GGML_TYPES.get(self.ggml_type)
        return t.what if t is not None and t.load == "blocks" else None


GGUFTensorInfo = TensorEntry  # the descriptor's name on the reference side

_VT_STRING, _VT_ARRAY = 8, 9
# metadata scalar value types: GGUF id -> numpy dtype (little endian)
_VT_SCALAR = {0: "<u1", 1: "<i1", 2: "<u2", 3: "<i2", 4: "<u4", 5: "<i4", 6: "<f4", 7: "?", 10: "<u8", 11: "<i8",
              12: "<f8"}
_HEADER = struct.Struct("<4sIQQ")
_U32, _U64 = struct.Struct("<I"), struct.Struct("<Q")


def scan(buf, size: int, path: str) -> dict:
    """Walk the container once. Returns version, metadata (key -> value),
    metadata_types (key -> type id, or (9, element type id) for arrays),
    alignment, data_offset and the tensor entries in file order."""
    pos = 0

    def take(n: int, what: str) -> int:
        nonlocal pos
        if pos + n > size:
            raise GGUFFormatError(f"{path}: the file ends inside {what} (it needs bytes {pos}..{pos + n} of a "
                                  f"{size}-byte file)")
        start, pos = pos, pos + n
        return start

    def u32(what):
        return _U32.unpack_from(buf, take(4, what))[0]

    def u64(what):
        return _U64.unpack_from(buf, take(8, what))[0]

    def text(what):
        n = u64(f"the byte count of {what}")
        start = take(n, what)
        # surrogateescape keeps bytes that are not UTF-8 (some vocabularies hold them)
        return bytes(buf[start:start + n]).decode("utf-8", "surrogateescape")

    def scalar(vt, what):
        dt = np.dtype(_VT_SCALAR[vt])
        v = np.frombuffer(buf, dtype=dt, count=1, offset=take(dt.itemsize, what))[0]
        return bool(v) if vt == 7 else v.item()

    def value(vt, what):
        if vt in _VT_SCALAR:
            return scalar(vt, what), vt
        if vt == _VT_STRING:
            return text(what), vt
        if vt != _VT_ARRAY:
            raise GGUFFormatError(f"{path}: {what} has value type {vt}, which GGUF does not define")
        et = u32(f"the element type of {what}")
        n = u64(f"the length of {what}")
        if et in _VT_SCALAR:
            dt = np.dtype(_VT_SCALAR[et])
            start = take(n * dt.itemsize, f"the {n} elements of {what}")
            items = np.frombuffer(buf, dtype=dt, count=n, offset=start).tolist()
            return items, (_VT_ARRAY, et)
        if et == _VT_STRING:
            if n * 8 > size - pos:  # each string has at least its 8-byte count
                raise GGUFFormatError(f"{path}: {what} says it holds {n} strings; the {size - pos} bytes left "
                                      "cannot")
            return [text(f"{what}[{i}]") for i in range(n)], (_VT_ARRAY, et)
        if et == _VT_ARRAY:
            raise UnsupportedGGUF(f"{path}: {what} is an array of arrays; this reader stops at one level")
        raise GGUFFormatError(f"{path}: {what} has element type {et}, which GGUF does not define")

    if size < _HEADER.size:
        raise GGUFFormatError(f"{path}: {size} bytes -- shorter than the {_HEADER.size}-byte GGUF header")
    magic, version, n_tensors, n_kv = _HEADER.unpack_from(buf, take(_HEADER.size, "the header"))
    if magic != b"GGUF":
        raise GGUFFormatError(f"{path}: begins with {magic!r} where a GGUF file begins with b'GGUF'")
    if version not in (2, 3):
        swapped = struct.unpack("<I", struct.pack(">I", version))[0]
        if swapped in (1, 2, 3):
            raise UnsupportedGGUF(f"{path}: a big-endian GGUF file (version field {version:#010x}); this reader "
                                  "reads little-endian files")
        if version == 1:
            raise UnsupportedGGUF(f"{path}: GGUF v1 stores 32-bit counts; convert the model again with a current "
                                  "llama.cpp to get v3")
        raise UnsupportedGGUF(f"{path}: GGUF v{version}; this reader knows v2 and v3")
    # every metadata pair and every descriptor starts with an 8-byte string length
    if (n_tensors + n_kv) * 8 > size:
        raise GGUFFormatError(f"{path}: a header announcing {n_kv} metadata pairs and {n_tensors} tensors does "
                              f"not fit in {size} bytes")

    metadata, types = {}, {}
    for i in range(n_kv):
        key = text(f"metadata key {i}")
        if key in metadata:
            raise GGUFFormatError(f"{path}: duplicate metadata key {key!r}")
        metadata[key], types[key] = value(u32(f"the value type of {key!r}"), f"metadata {key!r}")
    align = metadata.get("general.alignment", 32)
    if isinstance(align, bool) or not isinstance(align, int) or align < 1 or (align & (align - 1)):
        raise GGUFFormatError(f"{path}: general.alignment must be a power of two, got {align!r}")

    raw_entries = []
    for i in range(n_tensors):
        name = text(f"the name of tensor {i}")
        nd = u32(f"the rank of {name!r}")
        if nd < 1 or nd > 4:
            raise GGUFFormatError(f"{path}: tensor {name!r} is {nd}-dimensional; GGUF tensors have 1 to 4 "
                                  "dimensions")
        ne = tuple(u64(f"extent {d} of {name!r}") for d in range(nd))
        raw_entries.append((name, ne, u32(f"the GGML type of {name!r}"), u64(f"the data offset of {name!r}")))
    data_offset = -(-pos // align) * align

    entries, seen = [], set()
    for name, ne, gtype, rel in raw_entries:
        if name in seen:
            raise GGUFFormatError(f"{path}: duplicate tensor name {name!r}")
        seen.add(name)
        if rel % align:
            raise GGUFFormatError(f"{path}: tensor {name!r} starts {rel} bytes into the data section, which breaks "
                                  f"its {align}-byte alignment")
        t = GGML_TYPES.get(gtype)
        nbytes = None
        if t is not None and t.block is not None:
            if ne[0] % t.block:
                raise GGUFFormatError(f"{path}: tensor {name!r} is {t.name} with rows of {ne[0]} elements, which "
                                      f"{t.block}-element blocks do not divide")
            count = 1
            for d in ne:
                count *= d
            nbytes = count // t.block * t.size
            if data_offset + rel + nbytes > size:
                raise GGUFFormatError(f"{path}: tensor {name!r} needs bytes up to {data_offset + rel + nbytes}, but "
                                      f"the file stops at {size} (cut short?)")
        entries.append(TensorEntry(name, gtype, ne, data_offset + rel, nbytes))
    return {"version": version, "metadata": metadata, "metadata_types": types, "alignment": align,
            "data_offset": data_offset, "entries": entries}


class GGUFFile:
    """A GGUF file mapped read-only, usable as a context manager:

        with GGUFFile(path) as f:
            f.metadata["general.architecture"]
            f.tensors["blk.0.attn_q.weight"].shape
            f.tensor_bytes("blk.0.attn_q.weight")   # a view of the stored bytes
    """

    def __init__(self, path):
        self.path = os.fspath(path)
        with open(self.path, "rb") as fh:
            size = os.fstat(fh.fileno()).st_size
            if size == 0:
                raise GGUFFormatError(f"{self.path}: 0 bytes -- a GGUF file starts with a 24-byte header")
            self._map = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
        self.size = size
        try:
            found = scan(self._map, size, self.path)
        except BaseException:
            self.close()
            raise
        self.version = found["version"]
        self.metadata = found["metadata"]
        self.metadata_types = found["metadata_types"]
        self.alignment = found["alignment"]
        self.data_offset = found["data_offset"]
        self.tensors = {e.name: e for e in found["entries"]}

    def close(self):
        m, self._map = getattr(self, "_map", None), None
        if m is not None:
            m.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self, name) -> TensorEntry:
        try:
            return self.tensors[name]
        except KeyError:
            raise KeyError(f"{name!r}: no such tensor in {self.path}") from None

    def tensor_bytes(self, name, *, allow_unloaded: bool = False) -> memoryview:
        """The stored bytes of tensor `name` (a view of the map). A type this
        backend does not load raises its refusal unless `allow_unloaded`, for
        tools that copy such tensors through untouched."""
        e = self.info(name)
        why = refusal(e.ggml_type, name)
        if why is not None and not allow_unloaded:
            raise why
        if e.nbytes is None:
            raise why
        return memoryview(self._map)[e.offset:e.offset + e.nbytes]

    def __repr__(self):
        return f"<GGUFFile {self.path} v{getattr(self, 'version', '?')}: {len(getattr(self, 'tensors', {}))} tensors>"


def _rows_to_rotate_half(rows: np.ndarray, n_head: int, shape) -> np.ndarray:
    """llama.cpp's converter stores each head's q/k rows interleaved (row 2d + p
    holds rotary pair p of dimension d); the model expects the two halves one
    after the other (row p*dim + d). `rows` is [n_rows, bytes per row]: a row
    of blocks never spans rows, so whole rows move as they are."""
    n = rows.shape[0]
    if n_head <= 0 or n % (2 * n_head):
        raise UnsupportedGGUF(f"{n} rows of a {tuple(shape)} tensor do not split into {n_head} heads of rotary "
                              f"pairs (n_head={n_head})")
    per = n // (2 * n_head)
    return np.ascontiguousarray(rows.reshape(n_head, per, 2, -1).swapaxes(1, 2).reshape(n, -1))


def load_tensor(f: GGUFFile, name: str, keep_blocks: bool = False, permute_heads: int | None = None,
                device="hip"):
    """Tensor `name` of `f`, as the reference's `load_tensor`
    (gguf/__init__.py:135-170) returns it: F32, F16 and BF16 dense in their own
    dtype, bit for bit; q4_0, q8_0 and q4_k as a quantised tensor over the
    file's blocks (`keep_blocks=True`) or as their float32 dequantisation.
    `permute_heads=n` puts the q/k rows of n heads back in rotate-half order,
    moving whole rows."""
    from . import _C
    from .tensor import Tensor

    e = f.info(name)
    data = np.frombuffer(f.tensor_bytes(name), dtype=np.uint8)
    t = GGML_TYPES[e.ggml_type]
    if t.load == "dense":
        host = data.view({"float32": np.float32, "float16": np.float16, "bfloat16": np.uint16}[t.what])
        host = host.reshape(e.shape)
        if permute_heads is not None:
            host = _rows_to_rotate_half(host.reshape(e.shape[0], -1), permute_heads, e.shape).reshape(e.shape)
        return Tensor.from_numpy(np.array(host), dtype=t.what, device=device)
    if permute_heads is not None:
        data = _rows_to_rotate_half(data.reshape(e.shape[0], -1), permute_heads, e.shape).reshape(-1)
    q = _C._quantized_from_blob(data.tobytes(), e.shape, t.what, device=device)
    return q if keep_blocks else _C._dequantize(q)


def quantized_linear(f: GGUFFile, name: str, bias=None, device="hip"):
    """A QuantizedLinear over tensor `name`'s own blocks, as the reference's
    `quantized_linear` (gguf/__init__.py:173-201) builds one: the tensor must
    be a 2-D block tensor (out_features, in_features)."""
    from .quant import QuantizedLinear

    e = f.info(name)
    why = refusal(e.ggml_type, name)
    if why is not None:
        raise why
    if e.kind != "block":
        raise UnsupportedGGUF(f"tensor {name!r} is dense {e.type_name}; a QuantizedLinear needs block-quantised "
                              "weights (load a dense weight with load_tensor)")
    if len(e.shape) != 2:
        raise UnsupportedGGUF(f"tensor {name!r} has shape {e.shape}; a QuantizedLinear weight is "
                              "(out_features, in_features)")
    return QuantizedLinear(load_tensor(f, name, keep_blocks=True, device=device), bias)
