"""GGUF checkpoints for the hip device: the container and the loaders that put
a file's tensors on the device.

Mirrors torchnative/python/torchnative/gguf: `GGUFFile` (reader.py:306-492),
the GGML type table and its refusals (reader.py:111-166), `load_tensor`
(__init__.py:135-170) and `quantized_linear` (__init__.py:173-201). As in the
reference, block tensors are never decoded or re-encoded on the way in: the
file's GGML blocks go byte for byte to `_quantized_from_blob`, which on this
backend splits them into the device's code and scale planes
(tn_q4_0_from_blob / tn_q8_0_from_blob / tn_q4_k_from_blob), so `_quantized_blob` of a loaded
weight returns the file's bytes.

The container is read with `mmap` and `struct` only. Layout (GGUF v2/v3,
little-endian): magic "GGUF", u32 version, u64 tensor count, u64 key/value
count; key/value pairs (string key, u32 value type, value); tensor descriptors
(string name, u32 n_dims, u64 ne[n_dims] fastest-varying first, u32 GGML type,
u64 data offset); padding to `general.alignment` (default 32); tensor data.
Strings are a u64 byte length and the bytes.
"""

from __future__ import annotations

import mmap
import os
import struct

import numpy as np

__all__ = ["GGUFFile", "GGUFTensorInfo", "GGML_TYPES", "GGUFFormatError", "UnsupportedGGUF", "type_name",
           "refusal", "load_tensor", "quantized_linear"]

_MAGIC = b"GGUF"
_DEFAULT_ALIGNMENT = 32
_MAX_DIMS = 4


class GGUFFormatError(ValueError):
    """The bytes are not a well-formed GGUF file."""


class UnsupportedGGUF(NotImplementedError):
    """A well-formed GGUF construct that is refused, with the reason."""


# Why a type is not loaded. The first four follow the reference's four refusal
# kinds (reader.py:83-108); the last is this backend's own: a block format the
# reference holds whose kernels the hip device does not have.
_WHY = {
    "activation": ("is an activation-side block format (the right-hand operand llama.cpp builds inside "
                   "vec_dot), never a stored weight; `_quantize` refuses it as a weight for the same reason."),
    "no_candle": ("has no candle GgmlDType, so the reference has no storage or kernel for it; re-quantise the "
                  "model to q8_0 or q4_0 for this backend."),
    "not_wired": "is a plain numeric type no checkpoint uses for weights; it is not wired and not guessed at.",
    "removed": "is a repacked layout ggml dropped from the file format; a file carrying it is not read.",
    "not_on_hip": ("is a block format the reference holds, but the hip device implements only q4_0, q8_0 and "
                   "q4_k blocks; re-quantise to one of them."),
}

# GGML type id -> (name, elements per block, bytes per block, kind, dtype / format / refusal key).
# Ids, block sizes and byte sizes are the file format's (ggml.c type_traits).
GGML_TYPES = {
    0: ("F32", 1, 4, "dense", "float32"),
    1: ("F16", 1, 2, "dense", "float16"),
    30: ("BF16", 1, 2, "dense", "bfloat16"),
    2: ("Q4_0", 32, 18, "block", "q4_0"),
    8: ("Q8_0", 32, 34, "block", "q8_0"),
    3: ("Q4_1", 32, 20, "refused", "not_on_hip"),
    6: ("Q5_0", 32, 22, "refused", "not_on_hip"),
    7: ("Q5_1", 32, 24, "refused", "not_on_hip"),
    10: ("Q2_K", 256, 84, "refused", "not_on_hip"),
    11: ("Q3_K", 256, 110, "refused", "not_on_hip"),
    12: ("Q4_K", 256, 144, "block", "q4_k"),
    13: ("Q5_K", 256, 176, "refused", "not_on_hip"),
    14: ("Q6_K", 256, 210, "refused", "not_on_hip"),
    9: ("Q8_1", 32, 36, "refused", "activation"),
    15: ("Q8_K", 256, 292, "refused", "activation"),
    16: ("IQ2_XXS", 256, 66, "refused", "no_candle"),
    17: ("IQ2_XS", 256, 74, "refused", "no_candle"),
    18: ("IQ3_XXS", 256, 98, "refused", "no_candle"),
    19: ("IQ1_S", 256, 50, "refused", "no_candle"),
    20: ("IQ4_NL", 32, 18, "refused", "no_candle"),
    21: ("IQ3_S", 256, 110, "refused", "no_candle"),
    22: ("IQ2_S", 256, 82, "refused", "no_candle"),
    23: ("IQ4_XS", 256, 136, "refused", "no_candle"),
    29: ("IQ1_M", 256, 56, "refused", "no_candle"),
    34: ("TQ1_0", 256, 54, "refused", "no_candle"),
    35: ("TQ2_0", 256, 66, "refused", "no_candle"),
    39: ("MXFP4", 32, 17, "refused", "no_candle"),
    24: ("I8", 1, 1, "refused", "not_wired"),
    25: ("I16", 1, 2, "refused", "not_wired"),
    26: ("I32", 1, 4, "refused", "not_wired"),
    27: ("I64", 1, 8, "refused", "not_wired"),
    28: ("F64", 1, 8, "refused", "not_wired"),
    31: ("Q4_0_4_4", None, None, "refused", "removed"),
    32: ("Q4_0_4_8", None, None, "refused", "removed"),
    33: ("Q4_0_8_8", None, None, "refused", "removed"),
    36: ("IQ4_NL_4_4", None, None, "refused", "removed"),
    37: ("IQ4_NL_4_8", None, None, "refused", "removed"),
    38: ("IQ4_NL_8_8", None, None, "refused", "removed"),
}


def type_name(ggml_type: int) -> str:
    t = GGML_TYPES.get(ggml_type)
    return t[0] if t else f"<unknown GGML type id {ggml_type}>"


def refusal(ggml_type: int, tensor_name: str | None = None):
    """The UnsupportedGGUF for a type that is not loaded here, else None."""
    where = f" (tensor {tensor_name!r})" if tensor_name else ""
    t = GGML_TYPES.get(ggml_type)
    if t is None:
        return UnsupportedGGUF(f"GGML type id {ggml_type}{where} is unknown to this reader; it is refused rather "
                               "than read as some other type.")
    if t[3] == "refused":
        return UnsupportedGGUF(f"GGML type {t[0]}{where} {_WHY[t[4]]}")
    return None


# GGUF metadata value types: id -> struct code (8 = string, 9 = array)
_SCALAR = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}
_STRING, _ARRAY = 8, 9


class ArrayValue(list):
    """A GGUF array value; `element_type` keeps the GGUF element type id."""

    def __init__(self, element_type, items):
        super().__init__(items)
        self.element_type = element_type


class GGUFTensorInfo:
    """One tensor descriptor. `shape` is in torch order (GGUF's `ne`
    reversed), so a linear weight stored as ne = [in, out] is (out, in).
    `offset` is absolute in the file; `nbytes` is None for a type of unknown
    size (listed, never read)."""

    __slots__ = ("name", "ggml_type", "ne", "shape", "offset", "nbytes", "n_elements")

    def __init__(self, name, ggml_type, ne, offset, nbytes, n_elements):
        self.name, self.ggml_type, self.ne = name, ggml_type, tuple(ne)
        self.shape = tuple(reversed(self.ne))
        self.offset, self.nbytes, self.n_elements = offset, nbytes, n_elements

    @property
    def type_name(self) -> str:
        return type_name(self.ggml_type)

    @property
    def kind(self) -> str:
        t = GGML_TYPES.get(self.ggml_type)
        return t[3] if t else "refused"

    @property
    def format(self):
        """The `_quantized_formats()` name of a block type loaded here, else None."""
        t = GGML_TYPES.get(self.ggml_type)
        return t[4] if t and t[3] == "block" else None

    def __repr__(self):
        return (f"GGUFTensorInfo({self.name!r}, {self.type_name}, shape={self.shape}, offset={self.offset}, "
                f"nbytes={self.nbytes})")


class _Parser:
    """Sequential little-endian reads over the mapped file, each bounds-checked."""

    def __init__(self, buf, size, path):
        self.buf, self.size, self.path, self.pos = buf, size, path, 0

    def need(self, n, what):
        if n < 0 or self.pos + n > self.size:
            raise GGUFFormatError(f"{self.path}: truncated -- {what} needs {n} bytes at offset {self.pos} of a "
                                  f"{self.size}-byte file")
        p = self.pos
        self.pos += n
        return p

    def unpack(self, code, what):
        size = struct.calcsize("<" + code)
        return struct.unpack_from("<" + code, self.buf, self.need(size, what))[0]

    def string(self, what):
        n = self.unpack("Q", f"the length of {what}")
        p = self.need(n, what)
        # surrogateescape: bytes that are not UTF-8 survive a round trip
        return bytes(self.buf[p:p + n]).decode("utf-8", "surrogateescape")

    def value(self, vtype, what, nested=False):
        if vtype in _SCALAR:
            return self.unpack(_SCALAR[vtype], what)
        if vtype == _STRING:
            return self.string(what)
        if vtype != _ARRAY:
            raise GGUFFormatError(f"{self.path}: {what} has unknown GGUF value type {vtype}")
        if nested:
            raise UnsupportedGGUF(f"{self.path}: {what} is an array of arrays, which this reader does not read")
        etype = self.unpack("I", f"the element type of {what}")
        count = self.unpack("Q", f"the element count of {what}")
        if count > self.size - self.pos:  # every element takes at least one byte
            raise GGUFFormatError(f"{self.path}: {what} claims {count} elements with {self.size - self.pos} "
                                  "bytes left")
        if etype in _SCALAR:
            code = _SCALAR[etype]
            p = self.need(struct.calcsize("<" + code) * count, what)
            return ArrayValue(etype, list(struct.unpack_from(f"<{count}{code}", self.buf, p)))
        return ArrayValue(etype, [self.value(etype, f"{what}[{i}]", nested=True) for i in range(count)])


class GGUFFile:
    """A GGUF file, memory-mapped read-only.

        with GGUFFile(path) as f:
            f.metadata["general.architecture"]
            f.tensors["blk.0.attn_q.weight"]   # GGUFTensorInfo
            f.raw("blk.0.attn_q.weight")       # the stored bytes
    """

    def __init__(self, path):
        self.path = os.fspath(path)
        self._fh = open(self.path, "rb")
        self._mm = None
        try:
            self.size = os.fstat(self._fh.fileno()).st_size
            if self.size == 0:
                raise GGUFFormatError(f"{self.path}: empty file, not GGUF")
            self._mm = mmap.mmap(self._fh.fileno(), 0, access=mmap.ACCESS_READ)
            self._read_header()
        except BaseException:
            self.close()
            raise

    def close(self):
        if self._mm is not None:
            self._mm.close()
            self._mm = None
        if self._fh is not None:
            self._fh.close()
            self._fh = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _read_header(self):
        p = _Parser(self._mm, self.size, self.path)
        p0 = p.need(4, "the magic")
        magic = bytes(self._mm[p0:p0 + 4])
        if magic != _MAGIC:
            raise GGUFFormatError(f"{self.path}: not a GGUF file (magic {magic!r}, expected {_MAGIC!r})")
        version = p.unpack("I", "the version")
        if version not in (2, 3):
            if struct.unpack(">I", struct.pack("<I", version))[0] in (1, 2, 3):
                raise UnsupportedGGUF(f"{self.path}: big-endian GGUF (the version field reads {version:#x}); only "
                                      "little-endian files are read")
            if version == 1:
                raise UnsupportedGGUF(f"{self.path}: GGUF version 1 (32-bit counts) is not read; re-convert the "
                                      "model with a current llama.cpp")
            raise UnsupportedGGUF(f"{self.path}: GGUF version {version} is not read (2 and 3 are)")
        self.version = version
        n_tensors = p.unpack("Q", "the tensor count")
        n_kv = p.unpack("Q", "the metadata count")
        if 8 * max(n_tensors, n_kv) > self.size:  # every entry starts with an 8-byte length
            raise GGUFFormatError(f"{self.path}: the header claims {n_kv} metadata entries and {n_tensors} "
                                  f"tensors, more than {self.size} bytes can hold")
        self.metadata, self.metadata_types = {}, {}
        for i in range(n_kv):
            key = p.string(f"metadata key #{i}")
            vtype = p.unpack("I", f"the value type of {key!r}")
            if key in self.metadata:
                raise GGUFFormatError(f"{self.path}: metadata key {key!r} appears twice")
            self.metadata[key] = p.value(vtype, f"metadata {key!r}")
            self.metadata_types[key] = vtype
        align = self.metadata.get("general.alignment", _DEFAULT_ALIGNMENT)
        if type(align) is not int or align <= 0 or align & (align - 1):
            raise GGUFFormatError(f"{self.path}: general.alignment = {align!r} is not a positive power of two")
        self.alignment = align

        descs = []
        for i in range(n_tensors):
            name = p.string(f"tensor name #{i}")
            nd = p.unpack("I", f"the dimension count of {name!r}")
            if not 1 <= nd <= _MAX_DIMS:
                raise GGUFFormatError(f"{self.path}: tensor {name!r} has {nd} dimensions (1 to {_MAX_DIMS} allowed)")
            ne = [p.unpack("Q", f"dimension {d} of {name!r}") for d in range(nd)]
            gtype = p.unpack("I", f"the type of {name!r}")
            rel = p.unpack("Q", f"the data offset of {name!r}")
            descs.append((name, ne, gtype, rel))
        self.data_offset = (p.pos + align - 1) // align * align

        self.tensors = {}
        for name, ne, gtype, rel in descs:
            if name in self.tensors:
                raise GGUFFormatError(f"{self.path}: tensor {name!r} appears twice")
            if rel % align:
                raise GGUFFormatError(f"{self.path}: tensor {name!r} starts at data offset {rel}, not a multiple "
                                      f"of the alignment {align}")
            count = 1
            for d in ne:
                count *= d
            t = GGML_TYPES.get(gtype)
            nbytes = None
            if t is not None and t[1] is not None:
                if ne[0] % t[1]:
                    raise GGUFFormatError(f"{self.path}: tensor {name!r} is {t[0]} with ne[0] = {ne[0]}, not a "
                                          f"multiple of its block size {t[1]}")
                nbytes = count // t[1] * t[2]
                end = self.data_offset + rel + nbytes
                if end > self.size:
                    raise GGUFFormatError(f"{self.path}: tensor {name!r} ends at byte {end}, past the end of the "
                                          f"{self.size}-byte file (truncated)")
            self.tensors[name] = GGUFTensorInfo(name, gtype, ne, self.data_offset + rel, nbytes, count)

    def info(self, name) -> GGUFTensorInfo:
        if name not in self.tensors:
            raise KeyError(f"{self.path} has no tensor named {name!r}")
        return self.tensors[name]

    def raw(self, name, refuse=True) -> bytes:
        """The tensor's stored bytes. `refuse=False` returns the bytes of a
        type that is not loaded (size permitting), for tooling that copies
        tensors through untouched."""
        info = self.info(name)
        why = refusal(info.ggml_type, name)
        if refuse and why is not None:
            raise why
        if info.nbytes is None:
            raise why or UnsupportedGGUF(f"tensor {name!r}: {info.type_name} has no known byte size")
        return self._mm[info.offset:info.offset + info.nbytes]

    def __repr__(self):
        return (f"GGUFFile({self.path!r}, version={getattr(self, 'version', '?')}, "
                f"tensors={len(getattr(self, 'tensors', {}))}, metadata={len(getattr(self, 'metadata', {}))})")


def _unpermute_rows(rows: np.ndarray, n_head: int, shape) -> np.ndarray:
    """Undo llama.cpp's q/k row interleave (convert_hf_to_gguf's `permute`):
    within each head the file holds rows (d, p) in order d-major for pair
    index p in {0, 1}; HF's rotate-half layout wants p-major. `rows` is
    [n_rows, row_bytes] (whole rows: a row of blocks never mixes rows, so the
    blocks move as they are)."""
    n = rows.shape[0]
    if n_head <= 0 or n % (2 * n_head):
        raise UnsupportedGGUF(f"cannot undo the Llama q/k row permutation of shape {tuple(shape)} for "
                              f"n_head={n_head}")
    return np.ascontiguousarray(rows.reshape(n_head, n // (2 * n_head), 2, -1).transpose(0, 2, 1, 3)
                                .reshape(n, -1))


def load_tensor(f: GGUFFile, name: str, keep_blocks: bool = False, permute_heads: int | None = None,
                device="hip"):
    """One tensor of `f` (__init__.py:135-170 of the reference).

    F32/F16/BF16 come back dense in their own dtype, bit for bit. A q4_0 or
    q8_0 tensor comes back as a quantised tensor holding the file's blocks
    (`keep_blocks=True`) or as their float32 dequantisation on the device.
    `permute_heads` undoes llama.cpp's q/k row permutation for that many
    heads, moving whole rows of blocks."""
    from . import _C
    from .tensor import Tensor

    info = f.info(name)
    why = refusal(info.ggml_type, name)
    if why is not None:
        raise why
    raw = np.frombuffer(f.raw(name), dtype=np.uint8)
    if info.kind == "dense":
        dtype = GGML_TYPES[info.ggml_type][4]
        host = raw.view({"float32": np.float32, "float16": np.float16, "bfloat16": np.uint16}[dtype])
        host = host.reshape(info.shape)
        if permute_heads is not None:
            host = _unpermute_rows(host.reshape(info.shape[0], -1), permute_heads, info.shape).reshape(info.shape)
        return Tensor.from_numpy(host.copy(), dtype=dtype, device=device)
    if permute_heads is not None:
        raw = _unpermute_rows(raw.reshape(info.shape[0], -1), permute_heads, info.shape).reshape(-1)
    q = _C._quantized_from_blob(raw.tobytes(), info.shape, info.format, device=device)
    return q if keep_blocks else _C._dequantize(q)


def quantized_linear(f: GGUFFile, name: str, bias=None, device="hip"):
    """A QuantizedLinear whose weight is tensor `name`'s own blocks
    (__init__.py:173-201 of the reference): a 2-D block tensor
    (out_features, in_features); dense tensors are refused by name."""
    from .quant import QuantizedLinear

    info = f.info(name)
    if info.kind != "block":
        raise refusal(info.ggml_type, name) or UnsupportedGGUF(
            f"tensor {name!r} is {info.type_name}, not a block-quantised type; use load_tensor() for a dense "
            "weight")
    if len(info.shape) != 2:
        raise UnsupportedGGUF(f"tensor {name!r} has shape {info.shape}; a linear weight is 2-D")
    return QuantizedLinear(load_tensor(f, name, keep_blocks=True, device=device), bias)
