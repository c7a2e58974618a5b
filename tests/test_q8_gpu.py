"""q8_0 weights on the MI355X against the CPU oracle: bit for bit.

The q8_0 half of the reference's block-format tests (tests/numerics/test_q4ref.py
writer/reader cases, test_qgemm.py rows and lossless cases): llama.cpp's bytes
and bits for the codec, and the linear -- the GEMV for m <= 4 (two 16-byte
loads per block, v_dot4 on the int8 codes) and the integer-MFMA GEMM above --
equal to the oracle's restatement of BlockQ8_0::vec_dot_unopt
(k_quants.rs:738-757) with no tolerance.
"""

import struct

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


def _f32_list(hexstr):
    raw = bytes.fromhex(hexstr)
    return np.array(struct.unpack(f"<{len(raw) // 4}f", raw), dtype=np.float32)


def _qweight(tn, blob, n, k):
    return tn._quantized_from_blob(blob, (n, k), "q8_0", device="hip")


def test_golden_blobs_upload_dequantize_round_trip_and_requantise(tn, golden):
    cases, _ = golden
    seen = 0
    for (fmt, name), c in sorted(cases.items()):
        if fmt != "q8_0":
            continue
        shape = c["shape"] if len(c["shape"]) == 2 else [1, c["shape"][0]]
        blob = bytes.fromhex(c["blob"])
        q = _qweight(tn, blob, *shape)
        assert tn._quantized_blob(q) == blob, name
        assert tn._quantized_nbytes(q) == len(blob)
        assert tn._dequantize(q).numpy().reshape(-1).tobytes() == bytes.fromhex(c["dequant_f32"]), name
        x = _f32_list(c["input_f32"]).reshape(shape)
        w = tn._quantize(tn.tensor(x, device="hip"), "q8_0")
        assert tn._quantized_blob(w) == blob, name
        seen += 1
    assert seen == 2


def test_device_quantiser_matches_the_oracle_on_random_and_edge_blocks(tn):
    rng = np.random.default_rng(32)
    w = (rng.standard_normal((96, 256)) * 0.05).astype(np.float32)
    w[0, :32] = 0.0                                             # zero block: d = 0, id = 0
    w[1, :32] = np.linspace(-1, 1, 32, dtype=np.float32)        # symmetric extremes
    w[2, :32] = 1e-7                                            # subnormal f16 scale
    w[3, 5] = np.nan                                            # NaN: ignored by the max, code 0
    w[4, :32] = 1.0e7                                           # amax / 127 overflows f16 to inf
    w[5, :32] = np.concatenate([[127.0, -127.0], np.arange(30) - 14.5]).astype(np.float32)  # d = 1: x * id on .5 ties
    w[6, :32] = -np.arange(32, dtype=np.float32)                # the extreme is negative
    q = tn._quantize(tn.tensor(w, device="hip"), "q8_0")
    assert tn._quantized_blob(q) == O.q8_0_quantize(w)
    assert tn._dequantize(q).numpy().tobytes() == O.q8_0_dequantize(O.q8_0_quantize(w), w.size).tobytes()


@pytest.mark.parametrize("m,n,k,seed", [
    (1, 1536, 576, 1),                                    # BASELINE config 1's shape
    (1, 8, 64, 11), (3, 12, 512, 12), (2, 5, 1024, 13),   # test_q4ref.py shapes
    (4, 576, 1536, 2), (1, 49152, 576, 3),                # down-proj / lm_head shapes
    (1, 100, 32, 4), (1, 3, 16384, 5),                    # one block per row; the longest GEMV row
    (2, 7, 24576, 6),                                     # past the GEMV's items: the GEMM path
])
def test_linear_is_bit_identical_to_the_oracle(tn, m, n, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    blob = O.synth_q8_0_weight(n, k, 0.02, seed + 100)
    bias = rng.standard_normal(n).astype(np.float32) if seed % 2 else None
    want = O.q8_0_linear(x, blob, n, bias=bias, threads=8)
    b = tn.tensor(bias, device="hip") if bias is not None else None
    got = tn._quantized_linear(tn.tensor(x, device="hip"), _qweight(tn, blob, n, k), b).numpy()
    assert got.tobytes() == want.tobytes(), np.argwhere(got != want)[:5]


def test_scales_across_every_f16_regime(tn):
    """Weight scales over every finite f16 bit pattern, and activation
    blocks whose Q8_0 scale is below the smallest subnormal, subnormal, on
    the normal boundary and around the f16 maximum: dequantisation, the GEMV
    and the GEMM bit for bit against the oracle (a row whose activation scale
    rounds to inf gives the oracle's infinities and NaNs)."""
    k, nb = 1024, 32
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = bits[(bits & 0x7C00) != 0x7C00]
    n = len(finite) // nb
    rng = np.random.default_rng(42)
    blob = np.zeros((n * nb, 34), np.uint8)
    blob[:, :2] = finite[: n * nb].view(np.uint8).reshape(-1, 2)
    blob[:, 2:] = rng.integers(0, 256, size=(n * nb, 32), dtype=np.uint8)
    blob = blob.tobytes()
    q = _qweight(tn, blob, n, k)
    assert tn._dequantize(q).numpy().tobytes() == O.q8_0_dequantize(blob, n * k).tobytes()

    x = rng.standard_normal((6, k)).astype(np.float32)
    targets = [0.0, 1e-9, 2.9e-8, 5.9604645e-08, 8.9e-8, 6.097e-05, 6.1035156e-05, 6.104e-05, 1.0, 65504.0,
               65519.0, 65519.996]
    for i, t in enumerate(targets):
        blk = x[0, 32 * i:32 * (i + 1)]
        x[0, 32 * i:32 * (i + 1)] = (blk / np.max(np.abs(blk)) * np.float32(t * 127.0)).astype(np.float32)
    x[1, :32] *= np.float32(1e7)
    want = O.q8_0_linear(x, blob, n, threads=8)
    got = tn._quantized_linear(tn.tensor(x[:2], device="hip"), q).numpy()  # GEMV
    assert got[0].tobytes() == want[0].tobytes(), np.argwhere(got[0] != want[0])[:5]
    assert not np.isfinite(want[1]).any()
    assert np.array_equal(got[1], want[1], equal_nan=True)
    got6 = tn._quantized_linear(tn.tensor(x, device="hip"), q).numpy()  # m = 6: the GEMM
    assert np.array_equal(got6, want, equal_nan=True)
    assert got6[0].tobytes() == want[0].tobytes()


@pytest.mark.parametrize("m,n,k,seed", [
    (5, 11, 512, 21), (17, 10, 512, 22), (130, 9, 512, 23),  # test_qgemm.py row / tail counts
    (128, 256, 1024, 24), (200, 333, 576, 25), (512, 384, 4096, 26),
])
def test_gemm_is_bit_identical_to_the_oracle(tn, m, n, k, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) * 1.3).astype(np.float32)
    blob = O.synth_q8_0_weight(n, k, 0.01, seed + 100)
    bias = rng.standard_normal(n).astype(np.float32) if seed % 2 else None
    want = O.q8_0_linear(x, blob, n, bias=bias, threads=8)
    b = tn.tensor(bias, device="hip") if bias is not None else None
    got = tn._quantized_linear(tn.tensor(x, device="hip"), _qweight(tn, blob, n, k), b).numpy()
    assert got.tobytes() == want.tobytes(), np.argwhere(got != want)[:5]


def test_batched_rows_equal_one_row_calls_on_the_device(tn):
    rng = np.random.default_rng(177)
    k, n = 512, 11
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    q = tn._quantize(tn.tensor(w, device="hip"), "q8_0")
    for m in (2, 5, 17, 130):
        x = (rng.standard_normal((m, k)) * 1.3).astype(np.float32)
        batched = tn._quantized_linear(tn.tensor(x, device="hip"), q).numpy()
        rows = np.concatenate([tn._quantized_linear(tn.tensor(x[i:i + 1], device="hip"), q).numpy()
                               for i in range(m)])
        assert batched.tobytes() == rows.tobytes(), m


def test_lossless_operands_give_the_exact_integer_matmul(tn):
    rng = np.random.default_rng(1771)
    k = 64
    for n in (8, 9, 10, 11):
        codes = rng.integers(-127, 128, size=(n, k // 32, 32))
        blob = bytearray()
        for r in range(n):
            for b in range(k // 32):
                blob += struct.pack("<e", 1.0) + struct.pack("<32b", *codes[r, b])
        dense = codes.reshape(n, k)
        q = _qweight(tn, bytes(blob), n, k)
        for m in (2, 5, 17, 130):
            xs = rng.integers(-126, 127, size=(m, k))
            xs[:, 0], xs[:, 32] = 127, -127
            got = tn._quantized_linear(tn.tensor(xs.astype(np.float32), device="hip"), q).numpy()
            assert np.array_equal(got.astype(np.int64), xs @ dense.T)


def test_bf16_activations_and_output(tn):
    """bf16 in (widened exactly) and bf16 out (RNE of the f32 result), both
    paths, on a prefill-sized product checked on sampled rows."""
    rng = np.random.default_rng(5)
    m, k, n = 256, 2048, 3072
    xb = tn.tensor(rng.standard_normal((m, k)).astype(np.float32), dtype="bfloat16", device="hip")
    xw = xb.numpy()
    blob = O.synth_q8_0_weight(n, k, 0.01, 55)
    q = _qweight(tn, blob, n, k)
    ybits = tn._quantized_linear(xb, q, out_dtype="bfloat16").bits()
    rows = [0, 1, 127, 128, 255]
    assert np.array_equal(ybits[rows], O.bf16_from_f32(O.q8_0_linear(xw[rows], blob, n, threads=16)))
    y1 = tn._quantized_linear(tn.tensor(xw[3:4], dtype="bfloat16", device="hip"), q, out_dtype="bfloat16").bits()
    assert np.array_equal(y1[0], ybits[3])
