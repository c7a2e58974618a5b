"""q4_k weights on the MI355X against the CPU oracle: bit for bit.

The device writer must produce llama.cpp's quantize_row_q4_K_ref bytes on the
reference's writer fixtures (tests/golden/q4_k_writer.json) and the oracle's
bytes on random and edge blocks; the reader must give llama.cpp's bits for a
foreign blob; the linear (Q8_K activations, BlockQ4K::vec_dot_unopt,
k_quants.rs:1478-1558) must equal the oracle bit for bit at every row count,
with f32 or bf16 activations and outputs.
"""

import json
import os
import struct

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


def _qweight(tn, blob, n, k):
    return tn._quantized_from_blob(blob, (n, k), "q4_k", device="hip")


def test_writer_produces_llama_cpps_bytes_on_the_device(tn):
    with open(os.path.join(HERE, "golden", "q4_k_writer.json")) as fh:
        cases = json.load(fh)["cases"]
    for c in cases:
        x = np.frombuffer(bytes.fromhex(c["input_f32"]), dtype=np.float32).reshape(c["shape"])
        q = tn._quantize(tn.tensor(x, device="hip"), "q4_k")
        assert tn._quantized_blob(q) == bytes.fromhex(c["blob"]), c["name"]


def test_writer_matches_the_oracle_on_random_and_edge_blocks(tn):
    rng = np.random.default_rng(41)
    w = (rng.standard_normal((24, 1024)) * 0.02).astype(np.float32)
    w[0, :256] = 0.0                                   # all-zero super-block
    w[1, :32] = 0.25                                   # a constant sub-block (max == min)
    w[2, :256] = -np.abs(w[2, :256]) - 0.01            # negative only: min < 0, this_min clamps
    w[3, 256:512] = np.abs(w[3, 256:512]) + 0.5        # positive only: min reset to 0
    w[4, :32] *= 1e-4                                  # a sub-block whose 6-bit scale rounds to zero
    w[5, :256] = np.round(w[5, :256] * 400) / 8        # coarse values: ties in the searches
    w[6, 7] = 1e4                                      # one outlier sets the super-block's scale
    w[7, :256] *= 1e-7                                 # scales in the f16 subnormal range
    q = tn._quantize(tn.tensor(w, device="hip"), "q4_k")
    assert tn._quantized_blob(q) == O.q4_k_quantize(w)
    assert tn._dequantize(q).numpy().tobytes() == O.q4_k_dequantize(O.q4_k_quantize(w), w.size).tobytes()


def test_reader_round_trip_and_llama_cpps_bits(tn, golden):
    cases, _ = golden
    c = cases[("q4_k", "foreign")]
    blob = bytes.fromhex(c["blob"])
    shape = c["shape"] if len(c["shape"]) == 2 else [1, c["shape"][0]]
    q = _qweight(tn, blob, *shape)
    assert tn._quantized_blob(q) == blob and tn._quantized_nbytes(q) == len(blob)
    assert tn._dequantize(q).numpy().reshape(-1).tobytes() == bytes.fromhex(c["dequant_f32"])
    rnd = O.synth_q4_k_weight(40, 768, 3)
    q = _qweight(tn, rnd, 40, 768)
    assert tn._quantized_blob(q) == rnd
    assert tn._dequantize(q).numpy().tobytes() == O.q4_k_dequantize(rnd, 40 * 768).tobytes()


@pytest.mark.parametrize("m,n,k,seed", [
    (1, 8, 256, 11), (3, 12, 512, 12), (2, 5, 1024, 13),      # small, with 1-3 row tails
    (1, 1536, 576 // 64 * 256, 1), (4, 576, 1536, 2),         # decode-sized
    (1, 3000, 4096, 3), (1, 7, 14336, 4), (2, 9, 28672, 5),   # long rows
    (5, 33, 2048, 6), (17, 40, 512, 7), (64, 96, 1024, 8),    # more rows than one chunk
    (1, 3, 46080, 9), (3, 3, 46080, 10),                      # rows past the GEMV's LDS: the GEMM
])
def test_linear_is_bit_identical_to_the_oracle(tn, m, n, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    blob = O.synth_q4_k_weight(n, k, seed + 100)
    bias = rng.standard_normal(n).astype(np.float32) if seed % 2 else None
    want = O.q4_k_linear(x, blob, n, bias=bias, threads=8)
    b = tn.tensor(bias, device="hip") if bias is not None else None
    got = tn._quantized_linear(tn.tensor(x, device="hip"), _qweight(tn, blob, n, k), b).numpy()
    assert got.tobytes() == want.tobytes(), np.argwhere(got != want)[:5]


def test_scales_across_every_f16_regime_and_activation_extremes(tn):
    """d and dmin over every finite f16 bit pattern (two passes, d and dmin
    rotated), and activation super-blocks that are zero, hold a NaN, an
    infinity, ties of opposite sign, or values near the f32 limits: the
    dequantisation and the linear bit for bit (NaNs in the oracle's places)."""
    k, nsb = 1024, 4
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = bits[(bits & 0x7C00) != 0x7C00]
    n = len(finite) // nsb
    rng = np.random.default_rng(43)
    blob = rng.integers(0, 256, size=(n * nsb, 144), dtype=np.uint8)
    blob[:, 0:2] = finite[: n * nsb].view(np.uint8).reshape(-1, 2)
    blob[:, 2:4] = np.roll(finite[: n * nsb], 977).view(np.uint8).reshape(-1, 2)
    blob = blob.tobytes()
    q = _qweight(tn, blob, n, k)
    assert tn._dequantize(q).numpy().tobytes() == O.q4_k_dequantize(blob, n * k).tobytes()
    x = rng.standard_normal((4, k)).astype(np.float32)
    x[0, :256] = 0.0
    x[0, 300] = np.nan
    x[1, 5], x[1, 9] = 2.0, -2.0
    x[1, 600] = np.inf
    x[2, :256] *= np.float32(3e37)
    x[3, 256:512] *= np.float32(1e-38)
    x6 = np.concatenate([x, rng.standard_normal((2, k)).astype(np.float32)])
    want = O.q4_k_linear(x6, blob, n, threads=8)
    for m in (4, 6):  # the GEMV, then the MFMA GEMM
        got = tn._quantized_linear(tn.tensor(x6[:m], device="hip"), q).numpy()
        assert np.array_equal(got, want[:m], equal_nan=True), m
        fin = np.isfinite(want[:m])
        assert got[fin].tobytes() == want[:m][fin].tobytes(), m


def test_prefill_gemm_at_the_config3_shape(tn):
    """x bf16 [512, 4096] against W [14336, 4096] q4_k, bf16 out: sampled rows
    bit for bit against the oracle, and rows of a separate smaller call equal
    to the same rows of the full call."""
    rng = np.random.default_rng(3)
    m, k, n = 512, 4096, 14336
    xb = tn.tensor(rng.standard_normal((m, k)).astype(np.float32), dtype="bfloat16", device="hip")
    xw = xb.numpy()
    blob = O.synth_q4_k_weight(n, k, 33)
    q = _qweight(tn, blob, n, k)
    y32 = tn._quantized_linear(xb, q).numpy()
    rows = [0, 1, 31, 32, 255, 300, 511]
    assert y32[rows].tobytes() == O.q4_k_linear(xw[rows], blob, n, threads=16).tobytes()
    ybits = tn._quantized_linear(xb, q, out_dtype="bfloat16").bits()
    assert np.array_equal(O.bf16_from_f32(y32), ybits)
    part = tn._quantized_linear(tn.tensor(xw[300:309], device="hip"), q).numpy()
    assert part.tobytes() == y32[300:309].tobytes()


def test_lossless_operands_give_the_exact_integer_matmul(tn):
    rng = np.random.default_rng(11)
    n, k = 9, 512
    blob = bytearray()
    dense = np.zeros((n, k), np.int64)
    for r in range(n):
        for b in range(k // 256):
            sc, mn, nib = rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256)
            s = bytearray(12)
            for j in range(8):
                if j < 4:
                    s[j], s[j + 4] = sc[j], mn[j]
                else:
                    s[j + 4] = (sc[j] & 15) | ((mn[j] & 15) << 4)
                    s[j - 4] |= (sc[j] >> 4) << 6
                    s[j] |= (mn[j] >> 4) << 6
            qs = bytes(int(nib[64 * c + i] | (nib[64 * c + 32 + i] << 4)) for c in range(4) for i in range(32))
            blob += struct.pack("<ee", 1.0, 1.0) + bytes(s) + qs
            dense[r, 256 * b:256 * (b + 1)] = np.repeat(sc, 32) * nib - np.repeat(mn, 32)
    q = _qweight(tn, bytes(blob), n, k)
    for m in (1, 4, 7):
        xs = rng.integers(-126, 127, size=(m, k))
        xs[:, 0], xs[:, 256] = 127, 127
        got = tn._quantized_linear(tn.tensor(xs.astype(np.float32), device="hip"), q).numpy()
        assert np.array_equal(got.astype(np.int64), xs @ dense.T)


def test_batched_rows_equal_one_row_calls_and_bf16_io(tn):
    rng = np.random.default_rng(177)
    k, n = 1024, 70
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    q = tn._quantize(tn.tensor(w, device="hip"), "q4_k")
    x = (rng.standard_normal((13, k)) * 1.3).astype(np.float32)
    batched = tn._quantized_linear(tn.tensor(x, device="hip"), q).numpy()
    rows = np.concatenate([tn._quantized_linear(tn.tensor(x[i:i + 1], device="hip"), q).numpy() for i in range(13)])
    assert batched.tobytes() == rows.tobytes()
    xb = tn.tensor(x, dtype="bfloat16", device="hip")
    yb = tn._quantized_linear(xb, q, out_dtype="bfloat16").bits()
    want = O.q4_k_linear(xb.numpy(), tn._quantized_blob(q), n, threads=8)
    assert np.array_equal(yb, O.bf16_from_f32(want))
