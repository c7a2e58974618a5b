"""q4_0 on the MI355X against the CPU oracle: bit for bit.

Dequantised weights and quantiser bytes must equal llama.cpp's golden vectors;
the linear (GEMV for m <= 4, MFMA GEMM above) must equal the oracle's
restatement of the reference's x86_64 arithmetic bit for bit, at the
BASELINE configs' shapes and at the reference's own test shapes
(tests/numerics/test_q4ref.py, test_qgemm.py), and batched rows must equal
one-row calls.
"""

import struct

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    info = tn._hip_probe()  # refuses unless the device is a gfx950
    print("device:", info, flush=True)
    return tn


def _f32_list(hexstr):
    raw = bytes.fromhex(hexstr)
    return np.array(struct.unpack(f"<{len(raw) // 4}f", raw), dtype=np.float32)


def _qweight(tn, blob, n, k):
    return tn._quantized_from_blob(blob, (n, k), "q4_0", device="hip")


def test_golden_blobs_upload_dequantize_and_round_trip(tn, golden):
    cases, _ = golden
    for (fmt, name), c in sorted(cases.items()):
        if fmt != "q4_0":
            continue
        shape = c["shape"] if len(c["shape"]) == 2 else [1, c["shape"][0]]
        blob = bytes.fromhex(c["blob"])
        q = _qweight(tn, blob, *shape)
        assert tn._quantized_blob(q) == blob, name
        got = tn._dequantize(q).numpy().reshape(-1)
        assert got.tobytes() == bytes.fromhex(c["dequant_f32"]), name


def test_device_quantiser_writes_llama_cpp_bytes(tn, golden):
    cases, _ = golden
    for (fmt, name), c in sorted(cases.items()):
        if fmt != "q4_0" or "input_f32" not in c:
            continue
        x = _f32_list(c["input_f32"]).reshape(-1, c["shape"][-1])
        q = tn._quantize(tn.tensor(x, device="hip"), "q4_0")
        assert tn._quantized_blob(q) == bytes.fromhex(c["blob"]), name


def test_device_quantiser_matches_the_oracle_on_random_and_edge_blocks(tn):
    rng = np.random.default_rng(31)
    w = (rng.standard_normal((96, 256)) * 0.05).astype(np.float32)
    w[0, :32] = 0.0                                            # zero block
    w[1, :32] = np.linspace(-1, 1, 32, dtype=np.float32)       # opposite-sign extremes, first wins
    w[2, :32] = 1e-7                                           # subnormal f16 scale
    w[3, 5] = np.nan                                           # NaN never chosen as the extreme
    w[4, :32] = 1.0e6                                          # scale overflows f16 to inf
    q = tn._quantize(tn.tensor(w, device="hip"), "q4_0")
    assert tn._quantized_blob(q) == O.q4_0_quantize(w)


@pytest.mark.parametrize("m,n,k,seed", [
    (1, 1536, 576, 1),      # BASELINE config 1 (decode GEMV)
    (1, 8, 64, 11), (3, 12, 512, 12), (2, 5, 1024, 13),   # test_q4ref.py shapes
    (4, 576, 1536, 2), (1, 49152, 576, 3),                # SmolLM2-shaped down-proj / lm_head
    (1, 100, 32, 4), (1, 3, 16384, 5),                    # one block per row; a long row
    (1, 3, 24576, 7), (2, 3, 24608, 8),                   # the GEMV's longest row; one block more (GEMM)
])
def test_gemv_is_bit_identical_to_the_oracle(tn, m, n, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    blob = O.synth_q4_0_weight(n, k, 0.02, seed + 100)
    bias = rng.standard_normal(n).astype(np.float32) if seed % 2 else None
    want = O.q4_0_linear(x, blob, n, bias=bias, threads=8)
    q = _qweight(tn, blob, n, k)
    b = tn.tensor(bias, device="hip") if bias is not None else None
    got = tn._quantized_linear(tn.tensor(x, device="hip"), q, b).numpy()
    assert got.tobytes() == want.tobytes(), np.argwhere(got != want)[:5]


def test_gemv_scales_across_every_f16_regime(tn):
    """Weight scales over every finite f16 bit pattern (subnormals, both
    zeros, the largest normal) and activation blocks whose Q8_0 scale
    amax/127 lands below the smallest subnormal, among the subnormals, on
    the normal boundary and around the f16 maximum: dequantisation and the
    GEMV bit for bit against the oracle. In a row whose block scale overflows
    to inf the outputs are infinities and NaNs (inf - inf, 0 * inf) in the
    oracle's places."""
    k, nb = 1024, 32
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = bits[(bits & 0x7C00) != 0x7C00]
    n = len(finite) // nb
    rng = np.random.default_rng(41)
    blob = np.zeros((n * nb, 18), np.uint8)
    blob[:, :2] = finite[: n * nb].view(np.uint8).reshape(-1, 2)
    blob[:, 2:] = rng.integers(0, 256, size=(n * nb, 16), dtype=np.uint8)
    blob = blob.tobytes()
    q = _qweight(tn, blob, n, k)
    assert tn._dequantize(q).numpy().tobytes() == O.q4_0_dequantize(blob, n * k).tobytes()

    x = rng.standard_normal((2, k)).astype(np.float32)
    targets = [0.0, 1e-9, 2.9e-8, 5.9604645e-08, 8.9e-8, 6.097e-05, 6.1035156e-05, 6.104e-05, 1.0, 65504.0,
               65519.0, 65519.996]
    for i, t in enumerate(targets):
        blk = x[0, 32 * i:32 * (i + 1)]
        x[0, 32 * i:32 * (i + 1)] = (blk / np.max(np.abs(blk)) * np.float32(t * 127.0)).astype(np.float32)
    x[1, :32] *= np.float32(1e7)  # amax / 127 > 65520: the scale rounds to inf
    want = O.q4_0_linear(x, blob, n, threads=8)
    got = tn._quantized_linear(tn.tensor(x, device="hip"), q).numpy()
    assert got[0].tobytes() == want[0].tobytes(), np.argwhere(got[0] != want[0])[:5]
    assert not np.isfinite(want[1]).any()
    assert np.array_equal(got[1], want[1], equal_nan=True)
    # one row at a time takes the single-row kernel
    got0 = tn._quantized_linear(tn.tensor(x[:1], device="hip"), q).numpy()
    assert got0.tobytes() == want[:1].tobytes()


@pytest.mark.parametrize("m,n,k,seed", [
    (5, 11, 512, 21), (17, 10, 512, 22), (130, 9, 512, 23),  # test_qgemm.py row / tail counts
    (128, 256, 1024, 24), (200, 333, 576, 25), (512, 384, 4096, 26),
    # the tile shapes: 16 columns above, 32 columns (3 row tiles x 157), and
    # 128 x 128 (2 row tiles x 64, N not a multiple of 112)
    (300, 5000, 256, 27), (256, 8192, 256, 28),
])
def test_gemm_is_bit_identical_to_the_oracle(tn, m, n, k, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) * 1.3).astype(np.float32)
    blob = O.synth_q4_0_weight(n, k, 0.01, seed + 100)
    # odd seeds add a bias: the GEMM epilogue's addition, in every tile shape
    bias = rng.standard_normal(n).astype(np.float32) if seed % 2 else None
    want = O.q4_0_linear(x, blob, n, bias=bias, threads=8)
    b = tn.tensor(bias, device="hip") if bias is not None else None
    q = _qweight(tn, blob, n, k)
    got = tn._quantized_linear(tn.tensor(x, device="hip"), q, b).numpy()
    assert got.tobytes() == want.tobytes(), np.argwhere(got != want)[:5]
    # bf16 output: the f32 result narrowed RNE, in every tile shape
    gb = tn._quantized_linear(tn.tensor(x, device="hip"), q, b, out_dtype="bfloat16").bits()
    assert np.array_equal(gb, O.bf16_from_f32(want))


def test_batched_rows_equal_one_row_calls_on_the_device(tn):
    rng = np.random.default_rng(177)
    k, n = 512, 11
    blob = O.synth_q4_0_weight(n, k, 0.05, 178)
    q = _qweight(tn, blob, n, k)
    for m in (2, 5, 17, 130):
        x = (rng.standard_normal((m, k)) * 1.3).astype(np.float32)
        batched = tn._quantized_linear(tn.tensor(x, device="hip"), q).numpy()
        rows = np.concatenate([tn._quantized_linear(tn.tensor(x[i:i + 1], device="hip"), q).numpy()
                               for i in range(m)])
        assert batched.tobytes() == rows.tobytes(), m


def test_lossless_operands_give_the_exact_integer_matmul(tn):
    rng = np.random.default_rng(1770)
    k = 64
    for n in (8, 9, 10, 11):
        nib = rng.integers(0, 16, size=(n, k // 32, 32))
        blob = bytearray()
        for r in range(n):
            for b in range(k // 32):
                blob += struct.pack("<e", 1.0) + bytes(int(nib[r, b, j] | (nib[r, b, j + 16] << 4)) for j in range(16))
        dense = (nib - 8).reshape(n, k)
        q = _qweight(tn, bytes(blob), n, k)
        for m in (2, 5, 17, 130):
            xs = rng.integers(-126, 127, size=(m, k))
            xs[:, 0], xs[:, 32] = 127, -127
            got = tn._quantized_linear(tn.tensor(xs.astype(np.float32), device="hip"), q).numpy()
            assert np.array_equal(got.astype(np.int64), xs @ dense.T)


def test_config3_prefill_gemm_bf16_in_bf16_out_at_full_size(tn):
    """x bf16 [512, 4096], W [14336, 4096], bf16 out. The
    full product is checked bit for bit on a sample of rows (the oracle's cost
    is linear in rows; every row is an independent recurrence) and the whole
    output through the batched == per-row-chunk property."""
    rng = np.random.default_rng(3)
    m, k, n = 512, 4096, 14336
    xf = rng.standard_normal((m, k)).astype(np.float32)
    xb = tn.tensor(xf, dtype="bfloat16", device="hip")
    x_widened = xb.numpy()  # exact widening of the bf16 inputs
    blob = O.synth_q4_0_weight(n, k, 0.01, 33)
    q = _qweight(tn, blob, n, k)
    y = tn._quantized_linear(xb, q, out_dtype="bfloat16")
    ybits = y.bits()
    rows = [0, 1, 127, 128, 255, 300, 511]
    want32 = O.q4_0_linear(x_widened[rows], blob, n, threads=16)
    assert np.array_equal(ybits[rows], O.bf16_from_f32(want32))
    # f32 output of the same call narrows to the same bits
    y32 = tn._quantized_linear(xb, q).numpy()
    assert np.array_equal(O.bf16_from_f32(y32), ybits)
    # rows computed in a separate, smaller call are the same bits
    part = tn._quantized_linear(tn.tensor(x_widened[300:305], device="hip"), q).numpy()
    assert part.tobytes() == y32[300:305].tobytes()


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_gemm_prepass_aligned_and_unaligned_x_agree_bitwise(tn, fmt):
    """The GEMM's Q8_0 prepass has a 16-byte-load kernel for an aligned x and
    a per-element one for any other x; both give the same codes and scales,
    including a block of NaNs and a row of zeros, and match the oracle."""
    from torchnative_amd import _lib

    rng = np.random.default_rng(301)
    m, n, k = 37, 70, 1024
    x = (rng.standard_normal((m, k)) * 1.7).astype(np.float32)
    x[3, 64:96] = np.nan
    x[5] = 0.0
    blob = O.synth_q4_0_weight(n, k, 0.01, 302) if fmt == "q4_0" else O.synth_q8_0_weight(n, k, 0.01, 302)
    q = tn._quantized_from_blob(blob, (n, k), fmt, device="hip")
    want = (O.q4_0_linear if fmt == "q4_0" else O.q8_0_linear)(x, blob, n, threads=8)
    aligned = tn._quantized_linear(tn.tensor(x, device="hip"), q).numpy()
    # the same rows one float past a 16-byte boundary
    buf = tn.tensor(np.concatenate([np.zeros(1, np.float32), x.reshape(-1)]), device="hip")
    y = tn.empty((m, n), "float32", "hip")
    fn = getattr(_lib.lib(), f"tn_{fmt}_linear")
    _lib.check(fn(None, buf.data_ptr() + 4, _lib.TN_F32, m, k, *q._planes(), n, None, y.data_ptr(), _lib.TN_F32))
    unaligned = y.numpy()
    assert aligned.tobytes() == unaligned.tobytes()
    assert np.array_equal(aligned, want, equal_nan=True)
