"""The `format="f32"` exactness control on the device (quant.rs:273-279):
an f32 / f16 / bf16 "quantised" weight is stored element by element and
`_quantized_linear` on it is the dense linear on the widened weight, so the
two must agree to the bit. That checks the wiring (transpose convention, bias
broadcast, batch dimensions) apart from any rounding.

- the reference's own control test, mirrored (tests/_support/test_shim.py:
  13011-13061): integer-valued operands, where every order gives the exact
  integer sum, at k x m in (32, 4), (64, 3), (256, 2), with and without a
  bias and with a rank-3 input;
- random and ragged shapes: `_quantized_linear(x, _quantize(w, "f32"), b)`,
  `linear(x, w, b)` and the oracle's sequential fma chain (oracle.dense_linear,
  pinned on the CPU in test_oracle_dense.py) bit for bit;
- f16 / bf16: the stored bytes are half's round-to-nearest-even narrowing
  (the oracle's converters, special values included), `_dequantize` widens
  them exactly (a NaN quieted, as half's to_f32 does), and the linear equals
  the dense linear on the widened weight;
- the swap: `quantize_(model, "f32")` leaves a model's outputs bit-identical.
"""

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


def _dev(tn, a):
    return tn.tensor(np.ascontiguousarray(a, np.float32)).to("hip")


def _ints(rows, cols, amax, seed):
    return np.random.default_rng(seed).integers(-amax, amax + 1, (rows, cols)).astype(np.float32)


def _exact(x, w, b):
    out = x.astype(np.float64) @ w.T.astype(np.float64)  # integer-valued: exact in float64 too
    return out + b.astype(np.float64)[None, :]


@pytest.mark.parametrize("k,m", [(32, 4), (64, 3), (256, 2)])
def test_the_f32_control_on_integer_operands_is_exact(tn, k, m):
    w = _ints(m, k, 64, 1000 + k)
    x = _ints(3, k, 64, 1009 + k)
    b = np.array([float(i - m // 2) for i in range(m)], np.float32)
    qf = tn._quantize(_dev(tn, w), "f32")
    for bias in (None, b):
        got = tn._quantized_linear(_dev(tn, x), qf, None if bias is None else _dev(tn, bias)).numpy()
        want = _exact(x, w, np.zeros(m, np.float32) if bias is None else bias)
        assert np.array_equal(got.astype(np.float64), want), (k, m, bias is not None)
    got3 = tn._quantized_linear(_dev(tn, x.reshape(1, 3, k)), qf, _dev(tn, b)).numpy()
    assert got3.shape == (1, 3, m)
    assert np.array_equal(got3.reshape(3, m).astype(np.float64), _exact(x, w, b))


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (1, 576, 1536), (3, 15, 63), (5, 17, 65), (67, 576, 200),
                                   (130, 100, 7), (64, 64, 64), (2, 4096, 11)])
def test_f32_control_equals_linear_and_the_oracle_bit_for_bit(tn, m, k, n):
    rng = np.random.default_rng(m * 7919 + k * 31 + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    xd, wd, bd = _dev(tn, x), _dev(tn, w), _dev(tn, b)
    q = tn._quantize(wd, "f32")
    for bias, bdev in ((None, None), (b, bd)):
        got = tn._quantized_linear(xd, q, bdev).numpy()
        dense = tn._C.linear(xd, wd, bdev).numpy()
        want = O.dense_linear(x, w, bias)
        assert got.view(np.uint32).tobytes() == dense.view(np.uint32).tobytes(), "control != linear"
        assert got.view(np.uint32).tobytes() == want.view(np.uint32).tobytes(), "device != oracle chain"


def test_batched_rows_equal_one_row_calls(tn):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((70, 300)).astype(np.float32)
    w = rng.standard_normal((90, 300)).astype(np.float32)
    q = tn._quantize(_dev(tn, w), "f32")
    full = tn._quantized_linear(_dev(tn, x), q).numpy()
    for i in (0, 1, 63, 64, 69):
        one = tn._quantized_linear(_dev(tn, x[i:i + 1]), q).numpy()[0]
        assert np.array_equal(one.view(np.uint32), full[i].view(np.uint32)), i


def _specials():
    """f32 values that exercise the narrowing: ties, subnormals, overflow,
    infinities, NaNs with payloads, signed zeros."""
    bits = np.array([0x00000000, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00001, 0xffa00000, 0x7f800001,
                     0x3f800000, 0x3f801000, 0x3f803000, 0x3f800800, 0x477fe000, 0x477ff000, 0x47800000,
                     0x33800000, 0x33000000, 0x33000001, 0x387fc000, 0x38800000, 0x00000001, 0x7f7fffff,
                     0x3f808000, 0x3f818000, 0x3f80c000, 0xbf808001, 0x7f7f8000, 0x7f7f7fff], np.uint32)
    return bits.view(np.float32)


def _quiet_f16_widen(h):
    f = O.f16_to_f32(h)
    u = f.view(np.uint32).copy()
    nan = np.isnan(f)
    u[nan] |= 0x00400000  # half's to_f32: 0x7fc00000 | sign | payload << 13
    return u.view(np.float32)


def _quiet_bf16_widen(h):
    h = np.asarray(h, np.uint16).copy()
    nan = (h & 0x7FFF) > 0x7F80
    h[nan] |= 0x0040  # half's bf16 to_f32 quiets the same way
    return (h.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("fmt", ["f16", "bf16"])
def test_reduced_formats_store_half_narrowing_and_widen_exactly(tn, fmt):
    rng = np.random.default_rng(21)
    w = np.concatenate([_specials(), (rng.standard_normal(32 * 64 - _specials().size) * 3).astype(np.float32)])
    w = w.reshape(32, 64)
    q = tn._quantize(_dev(tn, w), fmt)
    blob = np.frombuffer(tn._quantized_blob(q), np.uint16).reshape(32, 64)
    want = O.f16_from_f32(w) if fmt == "f16" else O.bf16_from_f32(w)
    assert np.array_equal(blob, want.reshape(32, 64))
    assert tn._quantized_nbytes(q) == w.size * 2
    widened = tn._dequantize(q).numpy()
    exp = _quiet_f16_widen(want) if fmt == "f16" else _quiet_bf16_widen(want)
    assert np.array_equal(widened.view(np.uint32), exp.reshape(32, 64).view(np.uint32))


@pytest.mark.parametrize("fmt", ["f16", "bf16"])
def test_a_signalling_nan_from_a_blob_widens_quieted(tn, fmt):
    h = np.array([0x7C01, 0xFC01, 0x7E00, 0x3C00] if fmt == "f16" else [0x7F81, 0xFF81, 0x7FC0, 0x3F80],
                 np.uint16).repeat(8).reshape(1, 32)
    q = tn._quantized_from_blob(h.tobytes(), (1, 32), fmt, "hip")
    got = tn._dequantize(q).numpy().view(np.uint32)
    exp = (_quiet_f16_widen(h) if fmt == "f16" else _quiet_bf16_widen(h)).view(np.uint32)
    assert np.array_equal(got, exp)
    assert tn._quantized_blob(q) == h.tobytes()  # the bytes themselves move unchanged


@pytest.mark.parametrize("fmt", ["f16", "bf16"])
def test_reduced_format_linear_is_the_dense_linear_on_the_widened_weight(tn, fmt):
    rng = np.random.default_rng(31)
    x = rng.standard_normal((37, 576)).astype(np.float32)
    w = rng.standard_normal((129, 576)).astype(np.float32)
    b = rng.standard_normal(129).astype(np.float32)
    q = tn._quantize(_dev(tn, w), fmt)
    widened = tn._dequantize(q)
    got = tn._quantized_linear(_dev(tn, x), q, _dev(tn, b)).numpy()
    dense = tn._C.linear(_dev(tn, x), widened, _dev(tn, b)).numpy()
    want = O.dense_linear(x, widened.numpy(), b)
    assert np.array_equal(got.view(np.uint32), dense.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", ["f32", "f16", "bf16"])
def test_dense_blocks_move_byte_for_byte(tn, fmt):
    rng = np.random.default_rng(41)
    w = rng.standard_normal((12, 40)).astype(np.float32)
    q = tn._quantize(_dev(tn, w), fmt)
    blob = tn._quantized_blob(q)
    assert len(blob) == tn._quantized_nbytes(q) == w.size * (4 if fmt == "f32" else 2)
    if fmt == "f32":
        assert blob == w.tobytes()
    cpu = tn._quantized_to(q, "cpu")
    assert cpu.device == "cpu" and tn._quantized_blob(cpu) == blob
    back = tn._quantized_to(cpu, "hip")
    assert tn._quantized_blob(back) == blob
    assert tn._quantized_format(back) == fmt
    again = tn._quantized_from_blob(blob, (12, 40), fmt, "hip")
    assert np.array_equal(tn._dequantize(again).numpy().view(np.uint32),
                          tn._dequantize(q).numpy().view(np.uint32))


def test_quantize_to_f32_leaves_a_model_bit_identical(tn):
    from torchnative_amd.nn import Linear, Module

    class Block(Module):
        def __init__(self, rng):
            super().__init__()
            self.up = Linear(rng.standard_normal((96, 64)).astype(np.float32),
                             rng.standard_normal(96).astype(np.float32))
            self.down = Linear(rng.standard_normal((48, 96)).astype(np.float32))

        def forward(self, x):
            return self.down(self.up(x))

    rng = np.random.default_rng(51)
    model = Block(rng)
    x = _dev(tn, rng.standard_normal((2, 5, 64)).astype(np.float32))
    before = model.forward(x).numpy()
    report = tn.quantize_(model, "f32")
    assert len(report.replaced) == 2 and not report.skipped
    assert report.quantized_bytes == report.dense_bytes
    after = model.forward(x).numpy()
    assert after.shape == (2, 5, 48)
    assert np.array_equal(before.view(np.uint32), after.view(np.uint32))


def test_the_dense_control_refuses_other_activation_dtypes(tn):
    w = _dev(tn, np.ones((4, 32), np.float32))
    q = tn._quantize(w, "f32")
    xb = tn.tensor(np.ones((2, 32), np.float32), dtype="bfloat16").to("hip")
    with pytest.raises(NotImplementedError, match="dense control path"):
        tn._quantized_linear(xb, q)
    with pytest.raises(RuntimeError, match="mat1 and mat2 shapes cannot be multiplied"):
        tn._quantized_linear(_dev(tn, np.ones((2, 31), np.float32)), q)
