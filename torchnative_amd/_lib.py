"""ctypes binding of libtnhip.so (the C ABI declared in include/tnhip.h).

The library is required: if it is not built, importing a compute entry point
raises, naming the build command. Nothing here falls back to the host.
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtnhip.so")

TN_OK, TN_EINVAL, TN_ENOTIMPL, TN_EHIP, TN_EVALUE = 0, 1, 2, 3, 4
TN_F32, TN_BF16, TN_F16, TN_F64, TN_BOOL = 0, 1, 2, 3, 4
TN_PRO_NONE, TN_PRO_RMSNORM, TN_PRO_SILU, TN_PRO_RMSNORM_SILU = 0, 1, 2, 3

# every symbol include/tnhip.h declares, with (restype, argtypes)
_P, _I64, _I, _D, _SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double, ctypes.c_size_t


class Counters(ctypes.Structure):
    _fields_ = [
        ("dispatches", ctypes.c_uint64),
        ("bytes_uploaded", ctypes.c_uint64),
        ("host_downloads", ctypes.c_uint64),
        ("bytes_downloaded", ctypes.c_uint64),
        ("refusals", ctypes.c_uint64),
        ("workspace_bytes", ctypes.c_uint64),
    ]


class Q4Weight(ctypes.Structure):
    _fields_ = [("qs", ctypes.c_void_p), ("d", ctypes.c_void_p)]


class LlamaLayer(ctypes.Structure):
    _fields_ = [
        ("qkv", Q4Weight), ("o", Q4Weight), ("gate_up", Q4Weight), ("down", Q4Weight),
        ("ln1", ctypes.c_void_p), ("ln2", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
    ]


class Llama(ctypes.Structure):
    _fields_ = [
        ("n_layers", ctypes.c_int64), ("hidden", ctypes.c_int64), ("n_heads", ctypes.c_int64),
        ("n_kv_heads", ctypes.c_int64), ("head_dim", ctypes.c_int64), ("inter", ctypes.c_int64),
        ("vocab", ctypes.c_int64), ("cap", ctypes.c_int64), ("eps", ctypes.c_double),
        ("embed", ctypes.c_void_p), ("norm", ctypes.c_void_p), ("lm_head", Q4Weight),
        ("inv_freq", ctypes.c_void_p), ("layers", ctypes.POINTER(LlamaLayer)),
        ("prompt", ctypes.c_void_p), ("prompt_len", ctypes.c_int64),
        ("state", ctypes.c_void_p), ("tokens", ctypes.c_void_p), ("logits", ctypes.c_void_p),
        ("work", ctypes.c_void_p),
    ]


SIGNATURES = {
    "tn_last_error": (ctypes.c_char_p, []),
    "tn_abi_version": (_I, []),
    "tn_probe": (_I, [ctypes.c_char_p, _SZ]),
    "tn_counters": (_I, [ctypes.POINTER(Counters)]),
    "tn_counters_reset": (_I, []),
    "tn_ops": (ctypes.c_char_p, []),
    "tn_device_count": (_I, [ctypes.POINTER(_I)]),
    "tn_set_device": (_I, [_I]),
    "tn_get_device": (_I, [ctypes.POINTER(_I)]),
    "tn_malloc": (_I, [ctypes.POINTER(_P), _SZ]),
    "tn_free": (_I, [_P]),
    "tn_memcpy_h2d": (_I, [_P, _P, _SZ, _P]),
    "tn_memcpy_d2h": (_I, [_P, _P, _SZ, _P]),
    "tn_memcpy_d2d": (_I, [_P, _P, _SZ, _P]),
    "tn_memset": (_I, [_P, _I, _SZ, _P]),
    "tn_stream_create": (_I, [ctypes.POINTER(_P)]),
    "tn_stream_destroy": (_I, [_P]),
    "tn_stream_synchronize": (_I, [_P]),
    "tn_stream_begin_capture": (_I, [_P]),
    "tn_stream_end_capture": (_I, [_P, ctypes.POINTER(_P)]),
    "tn_device_synchronize": (_I, []),
    "tn_event_create": (_I, [ctypes.POINTER(_P)]),
    "tn_event_destroy": (_I, [_P]),
    "tn_event_record": (_I, [_P, _P]),
    "tn_event_synchronize": (_I, [_P]),
    "tn_event_elapsed_ms": (_I, [ctypes.POINTER(ctypes.c_float), _P, _P]),
    "tn_q4_0_from_blob": (_I, [_P, _P, _I64, _I64, _P, _P]),
    "tn_q4_0_to_blob": (_I, [_P, _P, _P, _I64, _I64, _P]),
    "tn_q4_0_quantize": (_I, [_P, _P, _I64, _I64, _P, _P]),
    "tn_q4_0_dequantize": (_I, [_P, _P, _P, _I64, _I64, _P]),
    "tn_q4_0_linear": (_I, [_P, _P, _I, _I64, _I64, _P, _P, _I64, _P, _P, _I]),
    "tn_q8_0_from_blob": (_I, [_P, _P, _I64, _I64, _P, _P]),
    "tn_q8_0_to_blob": (_I, [_P, _P, _P, _I64, _I64, _P]),
    "tn_q8_0_quantize": (_I, [_P, _P, _I64, _I64, _P, _P]),
    "tn_q8_0_dequantize": (_I, [_P, _P, _P, _I64, _I64, _P]),
    "tn_q8_0_linear": (_I, [_P, _P, _I, _I64, _I64, _P, _P, _I64, _P, _P, _I]),
    "tn_q4_k_from_blob": (_I, [_P, _P, _I64, _I64, _P]),
    "tn_q4_k_to_blob": (_I, [_P, _P, _I64, _I64, _P]),
    "tn_q4_k_quantize": (_I, [_P, _P, _I64, _I64, _P]),
    "tn_q4_k_dequantize": (_I, [_P, _P, _I64, _I64, _P]),
    "tn_q4_k_linear": (_I, [_P, _P, _I, _I64, _I64, _P, _I64, _P, _P, _I]),
    "tn_dense_quantize": (_I, [_P, _P, _I64, _I, _P]),
    "tn_dense_dequantize": (_I, [_P, _P, _I, _I64, _P]),
    "tn_dense_linear": (_I, [_P, _P, _I64, _I64, _P, _I, _I64, _P, _P]),
    "tn_q4_0_linear_decode": (_I, [_P, _P, _I64, _I, _P, _D, _P, _P, _I64, _P, _P]),
    "tn_sdpa_fwd": (_I, [_P, _I, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I, _P, _I, _D, _P, _P]),
    "tn_sdpa_decode": (_I, [_P, _I, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _D, _P, _P]),
    "tn_sdpa_decode_noalloc": (_I, [_P, _I, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _D, _P, _P]),
    "tn_embedding": (_I, [_P, _P, _I64, _P, _I64, _I64, _P]),
    "tn_rmsnorm": (_I, [_P, _P, _I64, _I64, _P, _D, _P]),
    "tn_rope": (_I, [_P, _P, _I64, _I64, _I64, _P, _P]),
    "tn_silu_mul": (_I, [_P, _P, _P, _I64, _P]),
    "tn_add": (_I, [_P, _P, _P, _I64, _P]),
    "tn_argmax": (_I, [_P, _P, _I64, _I64, _P]),
    "tn_kv_append": (_I, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "tn_llama_work_floats": (_I64, [ctypes.POINTER(Llama)]),
    "tn_llama_step": (_I, [_P, ctypes.POINTER(Llama)]),
    "tn_llama_capture": (_I, [_P, ctypes.POINTER(Llama), _I64, ctypes.POINTER(_P)]),
    "tn_llama_prefill_work_floats": (_I64, [ctypes.POINTER(Llama), _I64]),
    "tn_llama_prefill": (_I, [_P, ctypes.POINTER(Llama), _I64, _P]),
    "tn_graph_launch": (_I, [_P, _P]),
    "tn_graph_destroy": (_I, [_P]),
}

_lib = None
_lock = threading.Lock()


class HipLibraryMissing(RuntimeError):
    pass


def lib():
    """The loaded libtnhip.so. Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise HipLibraryMissing(
                f"torchnative_amd: {LIB_PATH} is not built; run `python -m torchnative_amd.build` "
                "(hipcc --offload-arch=gfx950). There is no host fallback."
            )
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().tn_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(status: int) -> None:
    """Map a tn_status onto the exception the reference raises (err.rs:11-28)."""
    if status == TN_OK:
        return
    msg = last_error()
    if status == TN_ENOTIMPL:
        raise NotImplementedError(msg)
    if status == TN_EVALUE:
        raise ValueError(msg)
    raise RuntimeError(msg)
