"""Dense tensors for the hip device: a device buffer plus shape and dtype.

This is the minimum a host needs to hand device pointers to the C ABI: the
reference's `TensorBase` (torchnative/rust/torch_c/src/tensor.rs) is a PyO3
object over candle storage; here a tensor is either host memory (a numpy
array, device "cpu") or a caller-owned HIP allocation (device "hip"). Compute
entry points accept only "hip" tensors and refuse the rest by name.
"""

from __future__ import annotations

import ctypes
import math
import weakref

import numpy as np

from . import _lib
from ._lib import check, lib

# name -> (numpy storage dtype, element size, C ABI dtype code or None)
DTYPES = {
    "float32": (np.float32, 4, _lib.TN_F32),
    "bfloat16": (np.uint16, 2, _lib.TN_BF16),
    "float16": (np.float16, 2, _lib.TN_F16),
    "float64": (np.float64, 8, _lib.TN_F64),
    "int32": (np.int32, 4, None),
    "int64": (np.int64, 8, None),
    "uint8": (np.uint8, 1, None),
    "bool": (np.bool_, 1, _lib.TN_BOOL),
}
float32, bfloat16, float16, float64 = "float32", "bfloat16", "float16", "float64"
int32, int64, uint8 = "int32", "int64", "uint8"

_current_stream = [None]


def current_stream():
    """The hipStream_t (as an int, or None for the default stream) calls go to."""
    return _current_stream[0]


class Stream:
    """A non-blocking HIP stream, usable as a context manager that makes it current."""

    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().tn_stream_create(ctypes.byref(p)))
        self.handle = p.value
        self._prev = []
        self._fin = weakref.finalize(self, _destroy_stream, self.handle)

    def synchronize(self):
        check(lib().tn_stream_synchronize(self.handle))

    def __enter__(self):
        self._prev.append(_current_stream[0])
        _current_stream[0] = self.handle
        return self

    def __exit__(self, *exc):
        _current_stream[0] = self._prev.pop()
        return False


def _destroy_stream(h):
    try:
        lib().tn_stream_destroy(h)
    except Exception:  # interpreter shutdown
        pass


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().tn_event_create(ctypes.byref(p)))
        self.handle = p.value
        self._fin = weakref.finalize(self, _destroy_event, self.handle)

    def record(self, stream=None):
        check(lib().tn_event_record(self.handle, stream if stream is not None else current_stream()))

    def synchronize(self):
        check(lib().tn_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().tn_event_elapsed_ms(ctypes.byref(ms), self.handle, end.handle))
        return float(ms.value)


def _destroy_event(h):
    try:
        lib().tn_event_destroy(h)
    except Exception:
        pass


def synchronize():
    check(lib().tn_device_synchronize())


class _DeviceBuffer:
    __slots__ = ("ptr", "nbytes", "__weakref__", "_fin")

    def __init__(self, nbytes: int):
        p = ctypes.c_void_p()
        check(lib().tn_malloc(ctypes.byref(p), int(nbytes)))
        self.ptr = p.value or 0
        self.nbytes = int(nbytes)
        self._fin = weakref.finalize(self, _free, self.ptr)


def _free(ptr):
    try:
        if ptr:
            lib().tn_free(ptr)
    except Exception:
        pass


def _parse_device(device) -> str:
    d = str(device)
    if d in ("cpu",):
        return "cpu"
    if d in ("hip", "hip:0", "cuda", "cuda:0"):
        return "hip"
    raise NotImplementedError(
        f"torchnative_amd: device {d!r} is not implemented; this backend knows 'cpu' (host memory, no "
        "compute) and 'hip' (the current MI355X)"
    )


def bf16_bits_from_f32(a) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even, NaN quieted."""
    x = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    rounded = ((x + np.uint32(0x7FFF) + ((x >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    nan = (x & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    return np.where(nan, ((x >> 16) | np.uint32(0x40)).astype(np.uint16), rounded)


def bf16_bits_to_f32(bits) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


class Tensor:
    """A dense row-major tensor on "cpu" (numpy) or "hip" (device memory)."""

    def __init__(self, shape, dtype: str, device: str = "hip", *, _host=None, _buf=None):
        if dtype not in DTYPES:
            raise NotImplementedError(f"torchnative_amd: dtype {dtype!r} is not implemented")
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.device = _parse_device(device)
        self._host = _host
        self._buf = _buf
        if self.device == "hip" and _buf is None:
            self._buf = _DeviceBuffer(max(self.nbytes, 1))
        if self.device == "cpu" and _host is None:
            self._host = np.zeros(self.shape, dtype=DTYPES[dtype][0])

    # --- construction ---------------------------------------------------------------
    @classmethod
    def empty(cls, shape, dtype="float32", device="hip"):
        return cls(shape, dtype, device)

    @classmethod
    def from_numpy(cls, arr, dtype: str | None = None, device="cpu"):
        """Copy a numpy array. With dtype="bfloat16" a float array is rounded
        RNE; a uint16 array is taken as bf16 bit patterns."""
        arr = np.asarray(arr)
        if dtype is None:
            dtype = {np.dtype(np.float32): "float32", np.dtype(np.float64): "float64",
                     np.dtype(np.float16): "float16", np.dtype(np.int32): "int32",
                     np.dtype(np.int64): "int64", np.dtype(np.uint8): "uint8",
                     np.dtype(np.bool_): "bool"}.get(arr.dtype)
            if dtype is None:
                raise NotImplementedError(f"torchnative_amd: numpy dtype {arr.dtype} has no tensor dtype")
        if dtype == "bfloat16":
            host = arr.astype(np.uint16) if arr.dtype == np.uint16 else bf16_bits_from_f32(arr)
        else:
            host = np.ascontiguousarray(arr, dtype=DTYPES[dtype][0])
        t = cls(host.shape, dtype, "cpu", _host=np.ascontiguousarray(host))
        return t.to(device)

    # --- properties -----------------------------------------------------------------
    @property
    def numel(self) -> int:
        return int(math.prod(self.shape))

    @property
    def element_size(self) -> int:
        return DTYPES[self.dtype][1]

    @property
    def nbytes(self) -> int:
        return self.numel * self.element_size

    def data_ptr(self) -> int:
        if self.device != "hip":
            raise RuntimeError("torchnative_amd: data_ptr() of a cpu tensor is not a device pointer")
        return self._buf.ptr

    def dim(self) -> int:
        return len(self.shape)

    def __repr__(self):
        return f"Tensor(shape={self.shape}, dtype={self.dtype}, device={self.device})"

    # --- movement ---------------------------------------------------------------------
    def to(self, device) -> "Tensor":
        dev = _parse_device(device)
        if dev == self.device:
            return self
        if dev == "hip":
            t = Tensor(self.shape, self.dtype, "hip")
            src = np.ascontiguousarray(self._host)
            check(lib().tn_memcpy_h2d(t._buf.ptr, src.ctypes.data, self.nbytes, current_stream()))
            return t
        host = np.empty(self.shape, dtype=DTYPES[self.dtype][0])
        check(lib().tn_memcpy_d2h(host.ctypes.data, self._buf.ptr, self.nbytes, current_stream()))
        return Tensor(self.shape, self.dtype, "cpu", _host=host)

    def cpu(self) -> "Tensor":
        return self.to("cpu")

    def numpy(self) -> np.ndarray:
        """Host copy; bfloat16 is widened to float32 (exact)."""
        host = self.cpu()._host
        if self.dtype == "bfloat16":
            return bf16_bits_to_f32(host).reshape(self.shape)
        return host.copy()

    def bits(self) -> np.ndarray:
        """Host copy of the raw storage (bfloat16 as uint16 bit patterns)."""
        return self.cpu()._host.copy()

    def view(self, *shape) -> "Tensor":
        """Same storage, new shape (dense row-major only)."""
        shape = tuple(shape[0]) if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else shape
        if -1 in shape:
            known = math.prod(s for s in shape if s != -1)
            shape = tuple(self.numel // known if s == -1 else s for s in shape)
        if math.prod(shape) != self.numel:
            raise RuntimeError(f"shape {tuple(shape)} is invalid for input of size {self.numel}")
        if self.device == "cpu":
            return Tensor(shape, self.dtype, "cpu", _host=self._host.reshape(shape))
        return Tensor(shape, self.dtype, "hip", _buf=self._buf)

    reshape = view

    def zero_(self) -> "Tensor":
        if self.device == "cpu":
            self._host[...] = 0
        else:
            check(lib().tn_memset(self._buf.ptr, 0, self.nbytes, current_stream()))
        return self


def tensor(data, dtype: str | None = None, device="cpu") -> Tensor:
    return Tensor.from_numpy(np.asarray(data), dtype=dtype, device=device)


def empty(shape, dtype="float32", device="hip") -> Tensor:
    return Tensor(shape, dtype, device)


def zeros(shape, dtype="float32", device="hip") -> Tensor:
    return Tensor(shape, dtype, device).zero_()
