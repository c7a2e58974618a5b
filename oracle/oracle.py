"""ctypes front end of ``libtnref.so`` plus numpy closed forms (TEST INFRASTRUCTURE ONLY).

Reference paths cited below are relative to the torchnative checkout:
``K`` = ``torchnative/rust/vendor/candle-core/src/quantized/k_quants.rs``,
``A`` = ``torchnative/rust/torch_c/src/aten.rs``.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

__all__ = [
    "lib", "build", "QK", "Q4_0_BYTES", "Q8_0_BYTES",
    "f16_from_f32", "f16_to_f32", "bf16_from_f32", "bf16_to_f32",
    "q4_0_quantize", "q4_0_dequantize", "q8_0_quantize", "q8_0_dequantize",
    "vec_dot_q4_0_q8_0", "q4_0_linear", "vec_dot_q8_0_q8_0", "q8_0_linear", "sdpa", "sdpa_bf16",
    "q4_0_parts", "q8_0_parts", "exact_linear_q4_0", "exact_linear_q8_0", "synth_q8_0_weight",
    "q4_k_quantize", "q4_k_dequantize", "q8_k_quantize", "vec_dot_q4_k_q8_k", "q4_k_linear", "q4_k_parts",
    "q8_k_parts", "exact_linear_q4_k", "accumulation_k_q4_k", "synth_q4_k_weight", "gamma", "accumulation_k",
    "linear_bound", "sdpa_closed_form", "sdpa_det", "q8_0_ties", "signed_max_ties",
    "synth_q4_0_weight", "sdpa_tolerance", "dense_linear",
]

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtnref.so")
QK = 32
Q4_0_BYTES = 18
Q8_0_BYTES = 34
QK_K = 256
Q4_K_BYTES = 144
Q8_K_BYTES = 292
U32 = 2.0 ** -24
U64 = 2.0 ** -53

_lib = None


def build() -> str:
    """Compile ``libtnref.so`` with the committed Makefile."""
    subprocess.run(["make", "-s", "-B", "-C", HERE, "libtnref.so"], check=True)
    return LIB_PATH


def lib():
    """Load the oracle library, building it only if nothing is built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    P, I64, I, D = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
    L.tnref_f16_from_f32.restype = ctypes.c_uint16
    L.tnref_f16_from_f32.argtypes = [ctypes.c_float]
    L.tnref_f16_to_f32.restype = ctypes.c_float
    L.tnref_f16_to_f32.argtypes = [ctypes.c_uint16]
    for name in ("tnref_f32_to_f16_n", "tnref_f32_to_bf16_n", "tnref_bf16_to_f32_n",
                 "tnref_q4_0_quantize", "tnref_q4_0_dequantize",
                 "tnref_q8_0_quantize", "tnref_q8_0_dequantize"):
        getattr(L, name).argtypes = [P, I64, P] if "quant" in name else [P, P, I64]
        getattr(L, name).restype = None
    L.tnref_vec_dot_q4_0_q8_0.restype = ctypes.c_float
    L.tnref_vec_dot_q4_0_q8_0.argtypes = [I64, P, P]
    L.tnref_q4_0_linear.restype = I
    L.tnref_q4_0_linear.argtypes = [I64, I64, I64, P, P, P, P, I]
    L.tnref_vec_dot_q8_0_q8_0.restype = ctypes.c_float
    L.tnref_vec_dot_q8_0_q8_0.argtypes = [I64, P, P]
    L.tnref_q8_0_linear.argtypes = [I64, I64, I64, P, P, P, P, I]
    for name in ("tnref_q4_k_quantize", "tnref_q8_k_quantize"):
        getattr(L, name).argtypes = [P, I64, P]
    L.tnref_q4_k_dequantize.argtypes = [P, I64, P]
    L.tnref_vec_dot_q4_k_q8_k.restype = ctypes.c_float
    L.tnref_vec_dot_q4_k_q8_k.argtypes = [I64, P, P]
    L.tnref_q4_k_linear.argtypes = [I64, I64, I64, P, P, P, P, I]
    L.tnref_dense_linear.restype = None
    L.tnref_dense_linear.argtypes = [I64, I64, I64, P, P, P, P]
    for name in ("tnref_sdpa_f32", "tnref_sdpa_f64"):
        fn = getattr(L, name)
        fn.restype = I
        fn.argtypes = [I64] * 6 + [P, P, P, P, I, D, P, P, I]
    _lib = L
    return L


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# --- reduced floats ---------------------------------------------------------


def f16_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().tnref_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return np.array([lib().tnref_f16_to_f32(int(v)) for v in h.reshape(-1)],
                    dtype=np.float32).reshape(h.shape)


def bf16_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().tnref_f32_to_bf16_n(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


# --- codecs -----------------------------------------------------------------


def q4_0_quantize(x) -> bytes:
    """GGML Q4_0 blob of a float32 array whose size is a multiple of 32 (K:241-277)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % QK == 0
    out = np.empty(x.size // QK * Q4_0_BYTES, dtype=np.uint8)
    lib().tnref_q4_0_quantize(_p(x), x.size, _p(out))
    return out.tobytes()


def q4_0_dequantize(blob, n) -> np.ndarray:
    b = np.frombuffer(bytes(blob), dtype=np.uint8)
    assert b.size == n // QK * Q4_0_BYTES
    out = np.empty(n, dtype=np.float32)
    lib().tnref_q4_0_dequantize(_p(b), n, _p(out))
    return out


def q8_0_quantize(x) -> bytes:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % QK == 0
    out = np.empty(x.size // QK * Q8_0_BYTES, dtype=np.uint8)
    lib().tnref_q8_0_quantize(_p(x), x.size, _p(out))
    return out.tobytes()


def q8_0_dequantize(blob, n) -> np.ndarray:
    b = np.frombuffer(bytes(blob), dtype=np.uint8)
    assert b.size == n // QK * Q8_0_BYTES
    out = np.empty(n, dtype=np.float32)
    lib().tnref_q8_0_dequantize(_p(b), n, _p(out))
    return out


def vec_dot_q4_0_q8_0(k, w_row: bytes, xq_row: bytes) -> float:
    w = np.frombuffer(bytes(w_row), dtype=np.uint8)
    x = np.frombuffer(bytes(xq_row), dtype=np.uint8)
    return float(np.float32(lib().tnref_vec_dot_q4_0_q8_0(k, _p(w), _p(x))))


def q4_k_quantize(x) -> bytes:
    """BlockQ4K::from_float (K:1570-1654): 144-byte super-blocks of 256."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size // QK_K * Q4_K_BYTES, dtype=np.uint8)
    lib().tnref_q4_k_quantize(_p(x), x.size, _p(out))
    return out.tobytes()


def q4_k_dequantize(blob, n) -> np.ndarray:
    b = np.frombuffer(bytes(blob), dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    lib().tnref_q4_k_dequantize(_p(b), n, _p(out))
    return out


def q8_k_quantize(x) -> bytes:
    """BlockQ8K::from_float (K:2375-2413): 292-byte blocks of 256."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size // QK_K * Q8_K_BYTES, dtype=np.uint8)
    lib().tnref_q8_k_quantize(_p(x), x.size, _p(out))
    return out.tobytes()


def vec_dot_q4_k_q8_k(k, w_row: bytes, xq_row: bytes) -> float:
    w = np.frombuffer(bytes(w_row), dtype=np.uint8)
    x = np.frombuffer(bytes(xq_row), dtype=np.uint8)
    return float(np.float32(lib().tnref_vec_dot_q4_k_q8_k(k, _p(w), _p(x))))


def vec_dot_q8_0_q8_0(k, w_row: bytes, xq_row: bytes) -> float:
    w = np.frombuffer(bytes(w_row), dtype=np.uint8)
    x = np.frombuffer(bytes(xq_row), dtype=np.uint8)
    return float(np.float32(lib().tnref_vec_dot_q8_0_q8_0(k, _p(w), _p(x))))


def _linear(fn, block_bytes, x, w_blob, n, bias, threads):
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    m = x.size // k if k else 0
    w = np.frombuffer(bytes(w_blob), dtype=np.uint8)
    assert w.size == n * (k // QK) * block_bytes, "blob size does not match [N, K]"
    y = np.empty(x.shape[:-1] + (n,), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = fn(m, k, n, _p(x), _p(w), _p(b), _p(y), int(threads))
    assert rc == 0
    return y


def q4_0_linear(x, w_blob, n, bias=None, threads=1) -> np.ndarray:
    """``torch._C._quantized_linear`` restated: y = Q8_0(x) . W^T (+ bias).

    x is float32 [..., K]; the result is float32 [..., N]."""
    return _linear(lib().tnref_q4_0_linear, Q4_0_BYTES, x, w_blob, n, bias, threads)


def q8_0_linear(x, w_blob, n, bias=None, threads=1) -> np.ndarray:
    """The same with a Q8_0 weight blob (34-byte blocks, K:738-757)."""
    return _linear(lib().tnref_q8_0_linear, Q8_0_BYTES, x, w_blob, n, bias, threads)


def dense_linear(x, w, bias=None) -> np.ndarray:
    """x [..., K] . w[N, K]^T (+ bias) in float32, each output the sequential
    fmaf chain over k that tn_dense_linear declares (the reference's own
    matmul order, the gemm crate's, is not restated)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    k = x.shape[-1]
    n = w.shape[0]
    assert w.shape == (n, k)
    y = np.empty(x.shape[:-1] + (n,), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().tnref_dense_linear(x.size // k, k, n, _p(x), _p(w), _p(b), _p(y))
    return y


def q4_k_linear(x, w_blob, n, bias=None, threads=1) -> np.ndarray:
    """A Q4_K weight blob: Q8_K activations and BlockQ4K::vec_dot_unopt."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    m = x.size // k if k else 0
    w = np.frombuffer(bytes(w_blob), dtype=np.uint8)
    assert w.size == n * (k // QK_K) * Q4_K_BYTES, "blob size does not match [N, K]"
    y = np.empty(x.shape[:-1] + (n,), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    assert lib().tnref_q4_k_linear(m, k, n, _p(x), _p(w), _p(b), _p(y), int(threads)) == 0
    return y


# --- SDPA -------------------------------------------------------------------


def sdpa(q, k, v, mask=None, is_causal=False, scale=None, threads=1, dtype=np.float32):
    """The default path of A:10330-10423 in float32 or float64.

    Returns ``(out, lse)``. q [B,Hq,L,D], k/v [B,Hkv,S,D]; mask broadcastable
    to [B,Hq,L,S]."""
    dt = np.dtype(dtype)
    q = np.ascontiguousarray(q, dtype=dt)
    k = np.ascontiguousarray(k, dtype=dt)
    v = np.ascontiguousarray(v, dtype=dt)
    B, Hq, L, D = q.shape
    _, Hkv, S, _ = k.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    m = None
    if mask is not None:
        m = np.ascontiguousarray(np.broadcast_to(np.asarray(mask, dtype=dt), (B, Hq, L, S)))
    out = np.empty((B, Hq, L, D), dtype=dt)
    lse = np.empty((B, Hq, L), dtype=dt)
    fn = lib().tnref_sdpa_f64 if dt == np.float64 else lib().tnref_sdpa_f32
    rc = fn(B, Hq, Hkv, L, S, D, _p(q), _p(k), _p(v), _p(m), int(bool(is_causal)),
            float(scale), _p(out), _p(lse), int(threads))
    assert rc == 0
    return out, lse


def sdpa_bf16(q_bits, k_bits, v_bits, mask=None, is_causal=False, scale=None, threads=1):
    """bf16 inputs (as uint16 bit patterns): widened to f32 for the whole body,
    the output narrowed back to bf16 RNE, the lse kept f32 (A:10196-10206,
    A:10412). Returns ``(out_bits uint16, lse float32)``."""
    q = bf16_to_f32(q_bits)
    k = bf16_to_f32(k_bits)
    v = bf16_to_f32(v_bits)
    out, lse = sdpa(q, k, v, mask, is_causal, scale, threads)
    return bf16_from_f32(out), lse


# --- closed forms (numpy, independent of libtnref) ----------------------------


def q4_0_parts(blob, n, k):
    """(d float64 [n, nb], q int64 [n, nb, 32]) with element j / j+16 from the
    low / high nibble of byte j (K:219-239)."""
    raw = np.frombuffer(bytes(blob), dtype=np.uint8).reshape(n, k // QK, Q4_0_BYTES)
    d = raw[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    qs = raw[:, :, 2:]
    lo = (qs & 0x0F).astype(np.int64) - 8
    hi = (qs >> 4).astype(np.int64) - 8
    return d, np.concatenate([lo, hi], axis=2)


def q8_0_parts(blob, m, k):
    raw = np.frombuffer(bytes(blob), dtype=np.uint8).reshape(m, k // QK, Q8_0_BYTES)
    d = raw[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    q = raw[:, :, 2:].copy().view(np.int8).astype(np.int64)
    return d, q


def exact_linear_q4_0(xq_blob, w_blob, m, n, k):
    """(value, abs_sum, ref_err), each float64 [m, n]: the exact dyadic value of
    the quantised matmul from the two blobs. Every block term is exact in
    float64 (15 + 11 + 11 bits); only the summation rounds, by at most
    ``ref_err``."""
    dw, qw = q4_0_parts(w_blob, n, k)
    return _exact_linear(dw, qw, xq_blob, m, n, k)


def exact_linear_q8_0(xq_blob, w_blob, m, n, k):
    """The same for a Q8_0 weight: block integers up to 32 * 127 * 128 (20
    bits) times two 11-bit scales, still exact in float64."""
    dw, qw = q8_0_parts(w_blob, n, k)
    return _exact_linear(dw, qw, xq_blob, m, n, k)


def _exact_linear(dw, qw, xq_blob, m, n, k):
    dx, qx = q8_0_parts(xq_blob, m, k)
    ints = np.einsum("rbk,obk->rob", qx, qw)
    absints = np.einsum("rbk,obk->rob", np.abs(qx), np.abs(qw))
    scale = dx[:, None, :] * dw[None, :, :]
    terms = ints.astype(np.float64) * scale
    if m * n <= 4096:
        value = np.array([math.fsum(r) for r in terms.reshape(-1, terms.shape[-1])]).reshape(m, n)
        rel = U64
    else:
        nb = terms.shape[-1]
        value = terms.sum(axis=-1)
        rel = nb * U64 / (1.0 - nb * U64)
    abs_sum = (absints.astype(np.float64) * np.abs(scale)).sum(axis=2)
    return value, abs_sum, rel * abs_sum


def q4_k_parts(blob, n, k):
    """(d, dmin float64 [n, nb], sc, mn int64 [n, nb, 8], q int64 [n, nb, 256])
    straight from the bytes (K:153-159 layout; the 6-bit packing of
    get_scale_min_k4, utils.rs:50-60, written out independently)."""
    raw = np.frombuffer(bytes(blob), dtype=np.uint8).reshape(n, k // QK_K, Q4_K_BYTES)
    d = raw[..., 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    dmin = raw[..., 2:4].copy().view(np.float16).astype(np.float64)[..., 0]
    s = raw[..., 4:16].astype(np.int64)
    sc = np.concatenate([s[..., 0:4] & 63, (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)], axis=-1)
    mn = np.concatenate([s[..., 4:8] & 63, (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)], axis=-1)
    qs = raw[..., 16:].astype(np.int64).reshape(n, k // QK_K, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=3).reshape(n, k // QK_K, QK_K)
    return d, dmin, sc, mn, q


def q8_k_parts(blob, m, k):
    raw = np.frombuffer(bytes(blob), dtype=np.uint8).reshape(m, k // QK_K, Q8_K_BYTES)
    d = raw[..., 0:4].copy().view(np.float32).astype(np.float64)[..., 0]
    q = raw[..., 4:4 + QK_K].copy().view(np.int8).astype(np.int64)
    return d, q


def exact_linear_q4_k(xq_blob, w_blob, m, n, k):
    """(value, abs_sum, ref_err) float64 [m, n]: the exact value of
    sum over super-blocks of (d_w*d_x) * sum_j sc_j * <q8, nib>_j - (dmin_w*d_x)
    * sum_j m_j * sum(q8)_j, from the two blobs. Each super-block term is exact
    in float64 only to rounding of its products, which ref_err bounds."""
    d, dmin, sc, mn, q = q4_k_parts(w_blob, n, k)
    dx, qx = q8_k_parts(xq_blob, m, k)
    nb = k // QK_K
    qx8 = qx.reshape(m, nb, 8, 32)
    q8w = q.reshape(n, nb, 8, 32)
    dots = np.einsum("rbjk,objk->robj", qx8, q8w)               # per sub-block integer dots
    sums = qx8.sum(axis=-1)                                      # [m, nb, 8]
    ints = (dots * sc[None]).sum(-1)                             # sum_j sc_j * dot_j
    absints = (np.einsum("rbjk,objk->robj", np.abs(qx8), q8w) * sc[None]).sum(-1)
    mins = (sums[:, None] * mn[None]).sum(-1)                    # sum_j m_j * sum(q8)_j
    absmins = (np.abs(sums)[:, None] * mn[None]).sum(-1)
    dd = dx[:, None, :] * d[None]
    dm = dx[:, None, :] * dmin[None]
    terms = ints * dd - mins * dm
    value = terms.sum(-1)
    abs_sum = (absints * np.abs(dd) + absmins * np.abs(dm)).sum(-1)
    return value, abs_sum, nb * 4 * U64 * abs_sum


def accumulation_k_q4_k(k):
    """Roundings on a term's path in K:1478-1558: d_w*d_x, the product with
    aux32 or sumi, the addition into its lane (up to nb of them), and the
    final 8-lane sum and the addition to sumf: nb + 12 (spares included)."""
    return k // QK_K + 12


def gamma(kk):
    return kk * U32 / (1.0 - kk * U32)


def accumulation_k(k):
    """Roundings on a block term's path to the output in the x86_64 scalar
    path (K:312-329): ``(s * d_w)`` and ``* d_x`` round once each; the
    sequential sum passes a term through at most nb-1 additions. Counted as
    nb + 2 (one spare)."""
    return k // QK + 2


def linear_bound(k, abs_sum, ref_err):
    return gamma(accumulation_k(k)) * abs_sum + ref_err


def sdpa_closed_form(q, k, v, mask=None, is_causal=False, scale=None):
    """softmax(q k^T * scale + causal + mask) v and its logsumexp in float64,
    written from the mathematics with an explicit repeat_interleave of the
    key/value heads and an explicit upper-left triangular mask."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Hq, L, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    rep = Hq // Hkv
    kk = np.repeat(k, rep, axis=1)
    vv = np.repeat(v, rep, axis=1)
    s = np.einsum("bhld,bhsd->bhls", q, kk) * scale
    if is_causal:
        tri = np.tril(np.ones((L, S), dtype=bool))  # row i keeps keys 0..=i
        s = np.where(tri, s, -np.inf)
    if mask is not None:
        s = s + np.asarray(mask, np.float64)
    mx = s.max(axis=-1, keepdims=True)
    w = np.exp(s - mx)
    tot = w.sum(axis=-1, keepdims=True)
    out = np.einsum("bhls,bhsd->bhld", w / tot, vv)
    lse = (np.log(tot) + mx)[..., 0]
    return out, lse


def sdpa_det(n, seed):
    """``n`` values k/128, exact in bf16/f16/f32/f64: the reference test
    inputs' generator (tests/_support/test_shim.py:12103-12116)."""
    out, state = [], seed * 2654435761 % 2147483647
    for _ in range(n):
        state = (state * 1103515245 + 12345) % 2147483648
        out.append((state % 321 - 160) / 128.0)
    return out


def q8_0_ties(x):
    """Elements whose Q8_0 rounding lands on an exact .5 (where half-even and
    half-away disagree)."""
    f = np.float32
    xs = np.asarray(x, dtype=f).reshape(-1, QK)
    d = (np.abs(xs).max(axis=1) / f(127)).astype(f)
    inv = np.where(d == 0, f(0), f(1) / np.where(d == 0, f(1), d)).astype(f)
    v = (xs * inv[:, None]).astype(f)
    return int(np.sum(np.abs(v - np.floor(v)) == f(0.5)))


def signed_max_ties(x, block=QK):
    xs = np.asarray(x, dtype=np.float32).reshape(-1, block)
    ax = np.abs(xs)
    amax = ax.max(axis=1, keepdims=True)
    at = (ax == amax) & (amax > 0)
    return int(np.sum(np.any(at & (xs > 0), axis=1) & np.any(at & (xs < 0), axis=1)))


def synth_q4_0_weight(n, k, sigma, seed):
    """The synthetic weight of BASELINE configs 1/3/5 as a GGML blob: codes
    uniform in [-8, 7] stored as nib = code + 8, per-block d = f16_rne(|N(0,
    sigma)| / 7). Built directly in the format (no quantiser involved)."""
    rng = np.random.default_rng(seed)
    nb = k // QK
    codes = rng.integers(-8, 8, size=(n, nb, QK), dtype=np.int64)
    d = (np.abs(rng.standard_normal((n, nb))) * sigma / 7.0).astype(np.float32)
    dh = f16_from_f32(d)
    nib = (codes + 8).astype(np.uint8)
    packed = (nib[:, :, :16] | (nib[:, :, 16:] << 4)).astype(np.uint8)
    blob = np.empty((n, nb, Q4_0_BYTES), dtype=np.uint8)
    blob[:, :, 0] = (dh & 0xFF).astype(np.uint8)
    blob[:, :, 1] = (dh >> 8).astype(np.uint8)
    blob[:, :, 2:] = packed
    return blob.tobytes()


def synth_q8_0_weight(n, k, sigma, seed):
    """A Q8_0 weight blob built directly in the format: codes uniform in
    [-127, 127], per-block d = f16_rne(|N(0, sigma)| / 127)."""
    rng = np.random.default_rng(seed)
    nb = k // QK
    codes = rng.integers(-127, 128, size=(n, nb, QK), dtype=np.int64)
    d = (np.abs(rng.standard_normal((n, nb))) * sigma / 127.0).astype(np.float32)
    dh = f16_from_f32(d)
    blob = np.empty((n, nb, Q8_0_BYTES), dtype=np.uint8)
    blob[:, :, 0] = (dh & 0xFF).astype(np.uint8)
    blob[:, :, 1] = (dh >> 8).astype(np.uint8)
    blob[:, :, 2:] = codes.astype(np.int8).view(np.uint8)
    return blob.tobytes()


def synth_q4_k_weight(n, k, seed):
    """A Q4_K weight blob built directly in the format: random nibbles and
    6-bit scales and mins, d and dmin f16 of |N(0, 0.02)| / 63 and / 630."""
    rng = np.random.default_rng(seed)
    nb = k // QK_K
    blob = np.empty((n, nb, Q4_K_BYTES), dtype=np.uint8)
    d = (np.abs(rng.standard_normal((n, nb))) * 0.02 / 63).astype(np.float32)
    dmin = (np.abs(rng.standard_normal((n, nb))) * 0.002 / 63).astype(np.float32)
    blob[..., 0:2] = f16_from_f32(d).view(np.uint8).reshape(n, nb, 2)
    blob[..., 2:4] = f16_from_f32(dmin).view(np.uint8).reshape(n, nb, 2)
    blob[..., 4:] = rng.integers(0, 256, size=(n, nb, Q4_K_BYTES - 4), dtype=np.uint8)
    return blob.tobytes()


def sdpa_tolerance(ref32, ref64, kind="float32", p=None, got=None, vsum=None):
    """Per-element bound on |gpu - ref32| for one SDPA output tensor.

    The rule (docs/numerics/AGREE.md section 2 of the reference, applied per
    tensor): 4x the reference's own fp32-vs-fp64 distance, floored at 10 ulp
    (1.186e-6) of the tensor's scale. A 16-bit output (``kind`` "bfloat16" or
    "float16") adds:

    - one ulp of the output format (both sides round to it; the spacing is
      taken at max(|ref|, |got|), as a value just under a power of two may
      round up across it; f16 spacing stops shrinking at its subnormals);
    - when ``p`` is given, the P-narrowing term u * sum_j P_ij |V_jd| with u
      the format's unit roundoff (2^-8 bf16, 2^-11 f16): pass ``p`` = that
      sum, the attention output with |V|;
    - for f16, when ``vsum`` = sum_j |V_jd| over the attended keys is given,
      2^-25 * vsum: probabilities below 2^-14 round in f16's subnormal range,
      at most 2^-25 each, against a row sum of at least 1."""
    ref32 = np.asarray(ref32, np.float64)
    ref64 = np.asarray(ref64, np.float64)
    fin = np.isfinite(ref64)
    own = float(np.max(np.abs(ref32 - ref64)[fin])) if fin.any() else 0.0
    scale_ = float(np.max(np.abs(ref64[fin]))) if fin.any() else 0.0
    tol = max(4.0 * own, 1.186e-6 * scale_)
    tol = np.full(ref32.shape, tol)
    if kind in ("bfloat16", "float16"):
        mant, emin, tiny, u = (7, -126, 2.0 ** -133, 2.0 ** -8) if kind == "bfloat16" else \
            (10, -14, 2.0 ** -24, 2.0 ** -11)
        mag = np.abs(ref64) if got is None else np.maximum(np.abs(ref64), np.abs(np.asarray(got, np.float64)))
        e = np.maximum(np.floor(np.log2(np.where(mag > 0, mag, 1e-38))), emin)
        tol = tol + np.where(mag > 0, 2.0 ** (e - mant), tiny)
        if p is not None:
            tol = tol + u * np.asarray(p, np.float64)
        if kind == "float16" and vsum is not None:
            tol = tol + 2.0 ** -25 * np.asarray(vsum, np.float64)
    return tol
