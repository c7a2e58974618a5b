"""The C ABI library loads, exports every symbol include/tnhip.h declares, and
its host-side argument checks refuse by name with the reference's wording.
None of these calls reaches the GPU: every refusal happens before a HIP call.
"""

import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "tnhip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tn_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from torchnative_amd import _lib

    return _lib.lib()


def test_library_exports_every_declared_symbol(L):
    from torchnative_amd import _lib

    names = _declared_symbols()
    assert len(names) >= 30
    for name in names:
        assert hasattr(L, name), name
    # and the Python binding knows every one of them, with a signature
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_abi_version_and_op_list(L):
    assert L.tn_abi_version() == 2
    ops = L.tn_ops().decode()
    assert "torch._C._quantized_linear(q4_0)" in ops
    assert "torch._C._quantized_linear(q8_0)" in ops
    assert "aten._scaled_dot_product_flash_attention_for_cpu.default" in ops


def test_linear_refusals_use_the_reference_wording(L):
    from torchnative_amd import _lib

    # bf16/f32 only (quant.rs:299-306): float16 activation refused by name
    st = L.tn_q4_0_linear(None, None, _lib.TN_F16, 1, 64, None, None, 8, None, None, _lib.TN_F32)
    assert st == _lib.TN_ENOTIMPL
    assert "activation must be float32" in _lib.last_error()
    # K not a block multiple -> the shape error of quant.rs:326-331
    st = L.tn_q4_0_linear(None, None, _lib.TN_F32, 1, 33, None, None, 8, None, None, _lib.TN_F32)
    assert st == _lib.TN_EINVAL
    assert "mat1 and mat2 shapes cannot be multiplied" in _lib.last_error()
    # quantiser: last dim not a multiple of 32 (quant.rs:145-161)
    st = L.tn_q4_0_quantize(None, None, 4, 48, None, None)
    assert st == _lib.TN_ENOTIMPL
    assert "must have their last dim divisible by block size -- got 48" in _lib.last_error()
    # q8_0 entry points: the same refusals, naming their format
    st = L.tn_q8_0_linear(None, None, _lib.TN_F16, 1, 64, None, None, 8, None, None, _lib.TN_F32)
    assert st == _lib.TN_ENOTIMPL and "activation must be float32" in _lib.last_error()
    st = L.tn_q8_0_linear(None, None, _lib.TN_F32, 2, 40, None, None, 8, None, None, _lib.TN_F32)
    assert st == _lib.TN_EINVAL and "cannot be multiplied ([2, 40]" in _lib.last_error()
    for fn in (L.tn_q8_0_quantize, L.tn_q8_0_from_blob):
        assert fn(None, None, 4, 48, None, None) == _lib.TN_ENOTIMPL
        assert "q8_0 stores 32 elements per block" in _lib.last_error()
    # q4_k: 256-element super-blocks
    assert L.tn_q4_k_quantize(None, None, 4, 512 + 32, None) == _lib.TN_ENOTIMPL
    assert "q4_k stores 256 elements per block, so it must have their last dim divisible by block size -- got 544" \
        in _lib.last_error()
    st = L.tn_q4_k_linear(None, None, _lib.TN_F32, 2, 288, None, 8, None, None, _lib.TN_F32)
    assert st == _lib.TN_EINVAL and "cannot be multiplied ([2, 288]" in _lib.last_error()
    # an empty product (no rows, or no output columns) is a success that
    # touches no pointer, as an empty matmul returns an empty tensor
    for m, n in ((0, 8), (2, 0), (0, 0)):
        assert L.tn_q4_0_linear(None, None, _lib.TN_F32, m, 64, None, None, n, None, None, _lib.TN_F32) == _lib.TN_OK
        assert L.tn_q8_0_linear(None, None, _lib.TN_BF16, m, 64, None, None, n, None, None, _lib.TN_BF16) == _lib.TN_OK
        assert L.tn_q4_k_linear(None, None, _lib.TN_F32, m, 256, None, n, None, None, _lib.TN_F32) == _lib.TN_OK
    # ... but the shape check still comes first
    st = L.tn_q4_0_linear(None, None, _lib.TN_F32, 0, 33, None, None, 8, None, None, _lib.TN_F32)
    assert st == _lib.TN_EINVAL and "cannot be multiplied ([0, 33]" in _lib.last_error()
    assert L.tn_q4_k_from_blob(None, None, 4, 256, None) == _lib.TN_EVALUE
    assert L.tn_q8_0_dequantize(None, None, None, 4, 96, None) == _lib.TN_EVALUE  # null planes
    assert "null pointer" in _lib.last_error()
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.TN_ENOTIMPL)


def test_sdpa_refusals_name_the_reason(L):
    from torchnative_amd import _lib

    args = dict(B=1, Hq=9, Hkv=3, L=8, S=8, D=64)

    def call(dtype=_lib.TN_BF16, mask=None, mask_dtype=0, **kw):
        a = {**args, **kw}
        return L.tn_sdpa_fwd(None, dtype, None, None, None, a["B"], a["Hq"], a["Hkv"], a["L"], a["S"], a["D"],
                             mask, mask_dtype, None, 1, float("nan"), None, None)

    assert call(D=272) == _lib.TN_ENOTIMPL and "head_dim 272" in _lib.last_error()
    assert call(Hkv=4) == _lib.TN_ENOTIMPL and "do not divide" in _lib.last_error()
    assert call(S=0) == _lib.TN_ENOTIMPL and "zero key length" in _lib.last_error()
    assert call(dtype=99) == _lib.TN_EINVAL and "Expected data type" in _lib.last_error()
    assert call(dtype=_lib.TN_F64, mask=1, mask_dtype=_lib.TN_F32) == _lib.TN_ENOTIMPL
    assert "float32 attn_mask on a float64" in _lib.last_error()
    # the mask is the query's dtype or float32 (aten.rs:10142-10150)
    assert call(mask=1, mask_dtype=_lib.TN_F16) == _lib.TN_EINVAL
    assert "Attention mask is the same data type as query" in _lib.last_error()
    assert call(dtype=_lib.TN_F32, mask=1, mask_dtype=_lib.TN_BF16) == _lib.TN_EINVAL
    assert call(dtype=_lib.TN_F16, mask=1, mask_dtype=_lib.TN_BF16) == _lib.TN_EINVAL
    # empty batch: nothing to write, success without touching a pointer
    assert call(B=0) == _lib.TN_OK
    assert call(L=0) == _lib.TN_OK  # no query rows (aten.rs:10242-10259)
    assert call(L=0, dtype=_lib.TN_F32, mask=1, mask_dtype=_lib.TN_BOOL) == _lib.TN_OK
    assert call(Hq=0, Hkv=3) == _lib.TN_OK  # 0 % 3: divisible, and nothing to write
    st = L.tn_sdpa_decode(None, _lib.TN_BF16, None, None, None, 2, 32, 8, 64, 128, None, 65, float("nan"),
                          None, None)
    assert st == _lib.TN_EINVAL and "max_len" in _lib.last_error()


def test_counters_shape_and_refusal_count(L):
    import torchnative_amd as tn

    tn._C._hip_counters_reset()
    before = tn._hip_counters()
    assert set(before) == {"dispatches", "bytes_uploaded", "host_downloads", "bytes_downloaded", "refusals",
                           "workspace_bytes"}
    from torchnative_amd import _lib

    L.tn_q4_0_quantize(None, None, 4, 48, None, None)
    assert tn._hip_counters()["refusals"] == before["refusals"] + 1


def test_python_mirror_refuses_host_operands_instead_of_falling_back():
    import torchnative_amd as tn

    x = tn.tensor(np.zeros((1, 64), np.float32))  # a cpu tensor
    with pytest.raises(NotImplementedError, match="does not fall back to the host"):
        tn._quantize(x, "q4_0")
    with pytest.raises(NotImplementedError, match="activation-side block format"):
        tn._quantize(x, "q8_1")
    with pytest.raises(ValueError, match="needs 18 bytes; got 17"):
        tn._quantized_from_blob(b"\0" * 17, (1, 32), "q4_0")
    with pytest.raises(ValueError, match="q8_0 stores 32 elements in 34 bytes.*needs 68 bytes; got 36"):
        tn._quantized_from_blob(b"\0" * 36, (1, 64), "q8_0")
    with pytest.raises(NotImplementedError, match="'q5_k' is not implemented on the hip device"):
        tn._quantize(x, "q5_k")
    assert tn._quantized_formats() == ["f32", "f16", "bf16", "q4_0", "q8_0", "q4_k"]
    with pytest.raises(ValueError, match="needs 256 bytes; got 128"):
        tn._quantized_from_blob(b"\0" * 128, (2, 32), "f32")
    qf = tn._quantized_from_blob(b"\0" * 128, (2, 32), "f16")  # host blob: 2 bytes per element, no compute
    assert tn._quantized_nbytes(qf) == 128 and tn._quantized_blob(qf) == b"\0" * 128
    q = tn._quantized_from_blob(b"\0" * 36, (1, 64), "q4_0")  # stays on the host: no compute
    assert tn._quantized_blob(q) == b"\0" * 36 and tn._quantized_nbytes(q) == 36
    with pytest.raises(NotImplementedError, match="hip device"):
        tn._quantized_linear(x, q)
    with pytest.raises(NotImplementedError, match="is not implemented for the hip device"):
        tn._aten_dispatch("aten.mm.default", x, x)
    with pytest.raises(RuntimeError, match="Currently do not support dropout > 0"):
        q4 = tn.tensor(np.zeros((1, 1, 2, 64), np.float32))
        tn._aten_dispatch("aten._scaled_dot_product_flash_attention_for_cpu.default", q4, q4, q4, 0.5)


def test_bf16_host_conversion_is_round_to_nearest_even():
    from torchnative_amd.tensor import bf16_bits_from_f32

    import oracle as O

    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32),
                        np.array([1.00390625, 1.005859375, np.inf, -np.inf, 0.0, -0.0], np.float32)])
    assert np.array_equal(bf16_bits_from_f32(x), O.bf16_from_f32(x))


def test_dense_format_refusals(L):
    from torchnative_amd import _lib

    # the dense formats are f32 / f16 / bf16 only; checked before any launch
    assert L.tn_dense_quantize(None, None, 8, _lib.TN_F64, None) == _lib.TN_ENOTIMPL
    assert "dense formats are f32, f16 and bf16" in _lib.last_error()
    assert L.tn_dense_dequantize(None, None, 99, 8, None) == _lib.TN_ENOTIMPL
    st = L.tn_dense_linear(None, None, 2, 0, None, _lib.TN_F32, 4, None, None)
    assert st == _lib.TN_EINVAL and "mat1 and mat2 shapes cannot be multiplied ([2, 0]" in _lib.last_error()
    assert L.tn_dense_linear(None, None, 2, 8, None, _lib.TN_F16, 4, None, None) == _lib.TN_EVALUE
    assert "null pointer" in _lib.last_error()
    assert L.tn_dense_linear(None, None, 0, 8, None, _lib.TN_BF16, 4, None, None) == _lib.TN_OK  # nothing to do


def test_fused_decode_linear_refusals(L):
    from torchnative_amd import _lib

    # checked on the host before anything reaches a device
    st = L.tn_q4_0_linear_decode(None, 4096, 64, 7, None, 0.0, 8192, 8192, 8, None, 16384)
    assert st == _lib.TN_EINVAL and "unknown prologue" in _lib.last_error()
    st = L.tn_q4_0_linear_decode(None, 4096, 64, _lib.TN_PRO_RMSNORM, None, 1e-5, 8192, 8192, 8, None, 16384)
    assert st == _lib.TN_EVALUE and "null pointer" in _lib.last_error()
    # y overlapping x ([gate | up] is 2k floats under the SiLU prologue)
    st = L.tn_q4_0_linear_decode(None, 4096, 64, _lib.TN_PRO_SILU, None, 0.0, 8192, 8192, 8, None, 4096 + 4 * 100)
    assert st == _lib.TN_EINVAL and "overlaps" in _lib.last_error()
