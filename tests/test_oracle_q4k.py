"""The Q4_K oracle (oracle/tnref.c), pinned without the reference's Rust.

* The writer (BlockQ4K::from_float, k_quants.rs:1570-1654) against the bytes of
  llama.cpp's quantize_row_q4_K_ref on the reference's own writer fixtures
  (tests/golden/q4_k_writer.json, made by tests/golden/make_q4_k_writer_vectors.py
  from the transcription in the reference's tests/numerics/test_q4kwriter.py).
* The reader (to_float, :1722-1746) against llama.cpp's bits for a foreign
  blob (tests/golden/golden_gguf_py.json, case q4_k/foreign).
* The Q8_K activation quantiser (:2375-2413) against its defining properties.
* The linear (vec_dot_unopt, :1478-1558) within the counted bound of the exact
  value computed from the two blobs; lossless operands give the exact
  integer matmul; batched rows equal one-row calls bit for bit.
"""

import json
import os
import struct

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))


def _writer_cases():
    with open(os.path.join(HERE, "golden", "q4_k_writer.json")) as fh:
        return json.load(fh)["cases"]


@pytest.mark.parametrize("case", _writer_cases(), ids=lambda c: c["name"])
def test_writer_produces_llama_cpps_bytes(case):
    x = np.frombuffer(bytes.fromhex(case["input_f32"]), dtype=np.float32)
    assert O.q4_k_quantize(x) == bytes.fromhex(case["blob"])


def test_writer_fixtures_cover_what_they_were_built_for():
    cases = {c["name"]: c for c in _writer_cases()}
    assert len(cases) == 11
    assert bytes.fromhex(cases["zeros"]["blob"]) == bytes(144)
    # a sub-block whose 6-bit scale rounds to zero keeps the search's levels:
    # its dequantised values are all -dmin*m (d*sc = 0), whatever its nibbles
    blob = bytes.fromhex(cases["zero_scale_sub"]["blob"])
    d, dmin, sc, mn, q = O.q4_k_parts(blob, 1, 256)
    assert sc[0, 0, 0] == 0 and q[0, 0, :32].any()


def test_reader_gives_llama_cpps_bits(golden):
    cases, _ = golden
    c = cases[("q4_k", "foreign")]
    n = int(np.prod(c["shape"]))
    assert O.q4_k_dequantize(bytes.fromhex(c["blob"]), n).tobytes() == bytes.fromhex(c["dequant_f32"])


def test_writer_round_trip_stays_within_its_levels():
    """Each element dequantises to within half a level step plus the 6-bit
    quantisation of its scale and min: a loose bound that a misplaced nibble,
    scale or min breaks by far."""
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((6, 1024)) * 0.02).astype(np.float32)
    blob = O.q4_k_quantize(w)
    dq = O.q4_k_dequantize(blob, w.size).reshape(w.shape)
    d, dmin, sc, mn, q = O.q4_k_parts(blob, 6, 1024)
    step = (d[..., None] * sc).repeat(32, axis=-1).reshape(w.shape)
    assert np.all(np.abs(dq - w) <= 2.0 * step + 1e-6)
    assert np.all((sc <= 63) & (mn <= 63)) and np.all((q >= 0) & (q <= 15))


def _q8k(x):
    raw = np.frombuffer(O.q8_k_quantize(x), dtype=np.uint8)
    d = raw[0:4].view(np.float32)[0]
    q = raw[4:260].view(np.int8).astype(np.int64)
    bs = raw[260:292].view(np.int16).astype(np.int64)
    return d, q, bs


def test_q8_k_activation_quantiser_properties():
    rng = np.random.default_rng(9)
    x = rng.standard_normal(256).astype(np.float32)
    x[17], x[200] = 3.5, -3.5                     # equal |x|, opposite signs: the first one wins
    d, q, bs = _q8k(x)
    iscale = np.float32(-127.0) / np.float32(3.5)
    assert q[17] == -127 and q[200] == 127
    assert d == np.float32(1.0) / iscale
    assert np.array_equal(q, np.clip(np.round(np.abs(iscale * x)) * np.sign(iscale * x), -128, 127))
    assert np.array_equal(bs, q.reshape(16, 16).sum(1))
    x[3] = np.nan                                  # never the extreme; its code is 0
    d2, q2, _ = _q8k(x)
    assert q2[3] == 0 and d2 == d
    dz, qz, bz = _q8k(np.zeros(256, np.float32))
    assert dz == 0 and not qz.any() and not bz.any()


@pytest.mark.parametrize("m,n,k,seed", [(1, 8, 256, 1), (3, 12, 1024, 2), (2, 5, 4096, 3)])
def test_linear_is_within_the_counted_bound_of_its_exact_value(m, n, k, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    blob = O.q4_k_quantize(w)
    got = O.q4_k_linear(x, blob, n).astype(np.float64)
    xq = b"".join(O.q8_k_quantize(r) for r in x)
    exact, abs_sum, ref_err = O.exact_linear_q4_k(xq, blob, m, n, k)
    bound = O.gamma(O.accumulation_k_q4_k(k)) * abs_sum + ref_err
    assert np.max(np.abs(got - exact) / bound) <= 1.0
    wdq = O.q4_k_dequantize(blob, n * k).astype(np.float64).reshape(n, k)
    assert np.max(np.abs(x.astype(np.float64) @ wdq.T - exact) / bound) > 1.0


def test_lossless_operands_give_the_exact_integer_matmul():
    """d = dmin = 1 and integer activations with absmax 127 per super-block
    (Q8_K: iscale = -1, codes = -x, d = -1): every step is exact, so the
    result is sum_j (sc_j * nib - m_j) . x, as integers."""
    rng = np.random.default_rng(11)
    n, k = 9, 512
    nb = k // 256
    blob = bytearray()
    dense = np.zeros((n, k), np.int64)
    for r in range(n):
        for b in range(nb):
            sc = rng.integers(0, 64, 8)
            mn = rng.integers(0, 64, 8)
            nib = rng.integers(0, 16, 256)
            s = bytearray(12)
            for j in range(8):
                if j < 4:
                    s[j] = sc[j]
                    s[j + 4] = mn[j]
                else:
                    s[j + 4] = (sc[j] & 15) | ((mn[j] & 15) << 4)
                    s[j - 4] |= (sc[j] >> 4) << 6
                    s[j] |= (mn[j] >> 4) << 6
            qs = bytes(int(nib[64 * c + i] | (nib[64 * c + 32 + i] << 4)) for c in range(4) for i in range(32))
            blob += struct.pack("<ee", 1.0, 1.0) + bytes(s) + qs
            dense[r, 256 * b:256 * (b + 1)] = (np.repeat(sc, 32) * nib - np.repeat(mn, 32))
    for m in (1, 4, 7):
        xs = rng.integers(-126, 127, size=(m, k))
        xs[:, 0], xs[:, 256] = 127, 127
        got = O.q4_k_linear(xs.astype(np.float32), bytes(blob), n, threads=2)
        assert np.array_equal(got.astype(np.int64), xs @ dense.T)


@pytest.mark.parametrize("m", [2, 5, 17])
def test_batched_rows_equal_one_row_calls_bit_for_bit(m):
    rng = np.random.default_rng(300 + m)
    k, n = 512, 11
    blob = O.q4_k_quantize((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    x = (rng.standard_normal((m, k)) * 1.3).astype(np.float32)
    batched = O.q4_k_linear(x, blob, n, threads=3)
    rows = np.concatenate([O.q4_k_linear(x[i:i + 1], blob, n) for i in range(m)])
    assert batched.tobytes() == rows.tobytes()
