"""Pins the CPU oracle's q4_0 / Q8_0 arithmetic before anything is compared to it.

Each check is chosen so that a plausible mistake in the restatement fails it:

* llama.cpp's own bytes and bits (``tests/golden/golden_gguf_py.json``, the
  reference's fixture ``scripts/q4quality/golden_gguf_py.json``, produced by
  gguf-py): writer and reader, no tolerance (reference test
  ``tests/numerics/test_q4ref.py:104-200``);
* the f16 conversion against numpy's IEEE binary16 conversion, exhaustively
  over every f16 and over f32 values at and around every rounding boundary;
* the linear against its exact dyadic value from the two blobs, under the
  counted Higham bound, and that bound refusing the matmul that skips
  activation quantisation (``test_q4ref.py:206-289``);
* batched rows == one-row calls bit for bit and lossless operands giving the
  exact integer matmul (``tests/numerics/test_qgemm.py:64-137``);
* planted faults (nibble pairing, unsigned scale, half-even rounding, f16 scale
  used for ``id``) made in a numpy copy of the algorithm must fail the same
  fixtures the oracle passes.
"""

import struct

import numpy as np
import pytest

import oracle as O


def _f32_list(hexstr):
    raw = bytes.fromhex(hexstr)
    return np.array(struct.unpack(f"<{len(raw) // 4}f", raw), dtype=np.float32)


# --- 1. llama.cpp's bytes and bits -----------------------------------------


def test_writers_produce_llama_cpp_bytes(golden):
    cases, _ = golden
    checked = 0
    for (fmt, name), c in sorted(cases.items()):
        if fmt not in ("q4_0", "q8_0") or "input_f32" not in c:
            continue
        x = _f32_list(c["input_f32"])
        got = O.q4_0_quantize(x) if fmt == "q4_0" else O.q8_0_quantize(x)
        assert got == bytes.fromhex(c["blob"]), (fmt, name)
        checked += 1
    assert checked == 9, f"expected 9 writer cases, found {checked}"


def test_readers_produce_llama_cpp_bits(golden):
    cases, _ = golden
    checked = 0
    for (fmt, name), c in sorted(cases.items()):
        if fmt not in ("q4_0", "q8_0"):
            continue
        n = int(np.prod(c["shape"]))
        blob = bytes.fromhex(c["blob"])
        got = O.q4_0_dequantize(blob, n) if fmt == "q4_0" else O.q8_0_dequantize(blob, n)
        assert got.tobytes() == bytes.fromhex(c["dequant_f32"]), (fmt, name)
        checked += 1
    assert checked == 9


def test_every_golden_case_still_exercises_its_edge(golden):
    """Fixture self-check, as test_q4ref.py:173-200 does: a trimmed or
    regenerated fixture must fail here rather than stop testing its edge."""
    cases, doc = golden
    assert len(doc["provenance"]["gguf_quants_sha256"]) == 64

    def d_of(c):
        return struct.unpack("<e", bytes.fromhex(c["blob"])[0:2])[0]

    assert d_of(cases[("q4_0", "pos_extreme")]) < 0
    assert d_of(cases[("q4_0", "neg_extreme")]) > 0
    zero = cases[("q4_0", "zero")]
    assert d_of(zero) == 0.0 and set(bytes.fromhex(zero["blob"])[2:]) == {0x88}
    opp = bytes.fromhex(cases[("q4_0", "opp_sign")]["blob"])[2:]
    nib = [b & 0xF for b in opp] + [b >> 4 for b in opp]
    assert nib[3] == 0 and nib[20] == 15
    raw = struct.unpack("<H", bytes.fromhex(cases[("q4_0", "subnormal_d")]["blob"])[0:2])[0]
    assert raw & 0x7C00 == 0 and raw & 0x3FF
    assert cases[("q4_0", "two_rows")]["shape"] == [2, 64]
    ties = _f32_list(cases[("q8_0", "ties")]["input_f32"])
    assert np.max(np.abs(ties)) == 127.0 and 2.5 in ties and -126.5 in ties


# --- 2. reduced floats ------------------------------------------------------


def test_f16_conversion_matches_ieee_binary16_exhaustively():
    # every f16 bit pattern widens exactly and narrows back to itself
    allh = np.arange(1 << 16, dtype=np.uint16)
    fin = (allh & 0x7C00) != 0x7C00
    wide = O.f16_to_f32(allh[fin])
    assert np.array_equal(wide.view(np.uint32), allh[fin].view(np.float16).astype(np.float32).view(np.uint32))
    assert np.array_equal(O.f16_from_f32(wide), allh[fin])
    # midpoints and their neighbours between consecutive f16 values: RNE ties
    lo = allh[fin][:-1].view(np.float16).astype(np.float64)
    hi = allh[fin][1:].view(np.float16).astype(np.float64)
    ok = np.isfinite(lo) & np.isfinite(hi) & (np.sign(lo) == np.sign(hi)) & (hi != lo)
    mid = ((lo[ok] + hi[ok]) / 2).astype(np.float32)
    probe = np.concatenate([mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(-np.inf))])
    want = probe.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f16_from_f32(probe), want)
    # random f32 over the whole range, including overflow to inf and underflow to 0
    rng = np.random.default_rng(5)
    r = rng.integers(0, 1 << 32, size=200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    r = r[np.isfinite(r)]
    with np.errstate(over="ignore"):
        want = r.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f16_from_f32(r), want)


def test_bf16_rounding_is_nearest_even_and_quiets_nan():
    # exact cases: values already in bf16 stay; ties go to even
    x = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, -2.5, 3.0e38, np.inf], dtype=np.float32)
    # 1 + 2^-8 is a tie between 1 and 1+2^-7 -> even (1.0); 1.005859375 = 1 + 3*2^-9 -> 1+2^-7
    want = np.array([0x3F80, 0x3F80, 0x3F81, 0x3F81, 0xC020, 0x7F62, 0x7F80], dtype=np.uint16)
    got = O.bf16_from_f32(x)
    assert np.array_equal(got, want), [hex(v) for v in got]
    snan = np.array([0x7F800001], dtype=np.uint32).view(np.float32)
    assert O.bf16_from_f32(snan)[0] == 0x7FC0
    # against float64 rounding to 8 significant bits, nearest-even, on random normals
    rng = np.random.default_rng(6)
    v = rng.standard_normal(100_000).astype(np.float32)
    m, e = np.frexp(v.astype(np.float64))
    r = np.ldexp(np.round(m * 256.0), e - 8).astype(np.float32)  # np.round is half-even
    assert np.array_equal(O.bf16_from_f32(v), (r.view(np.uint32) >> 16).astype(np.uint16))


# --- 3. the linear against its exact value ---------------------------------


def _tie_free(rows, cols, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, cols)) * 1.7).astype(np.float32)
    assert O.q8_0_ties(x) == 0 and O.signed_max_ties(x) == 0
    return x


@pytest.mark.parametrize("rows,out_f,in_f,seed", [(1, 8, 64, 11), (3, 12, 512, 12), (2, 5, 1024, 13), (1, 1536, 576, 14)])
def test_linear_is_within_the_counted_bound_of_its_exact_value(rows, out_f, in_f, seed):
    w = (np.random.default_rng(seed + 1).standard_normal((out_f, in_f)) * 0.05).astype(np.float32)
    x = _tie_free(rows, in_f, seed)
    blob = O.q4_0_quantize(w)
    got = O.q4_0_linear(x, blob, out_f).astype(np.float64)
    xq = O.q8_0_quantize(x)
    exact, abs_sum, ref_err = O.exact_linear_q4_0(xq, blob, rows, out_f, in_f)
    bound = O.linear_bound(in_f, abs_sum, ref_err)
    assert np.max(np.abs(got - exact) / bound) <= 1.0
    # the bound must refuse the nearest wrong matmul: no activation quantisation
    wdq = O.q4_0_dequantize(blob, out_f * in_f).astype(np.float64).reshape(out_f, in_f)
    wrong = x.astype(np.float64) @ wdq.T
    assert np.max(np.abs(wrong - exact) / bound) > 1.0


def test_the_bound_is_counted_not_chosen():
    assert O.accumulation_k(1024) == 1024 // 32 + 2
    k = O.accumulation_k(512)
    assert O.gamma(k) == k * 2.0 ** -24 / (1 - k * 2.0 ** -24)


def test_linear_matches_a_numpy_float32_restatement_bit_for_bit():
    """The scalar per-block recurrence of K:312-329 spelled in numpy float32
    (vectorised over outputs, sequential over blocks): bitwise equal."""
    rng = np.random.default_rng(21)
    m, k, n = 3, 256, 40
    x = rng.standard_normal((m, k)).astype(np.float32)
    blob = O.synth_q4_0_weight(n, k, 0.02, 22)
    dw, qw = O.q4_0_parts(blob, n, k)
    xq = O.q8_0_quantize(x)
    dx, qx = O.q8_0_parts(xq, m, k)
    ints = np.einsum("rbk,obk->rob", qx, qw)
    acc = np.zeros((m, n), np.float32)
    for b in range(k // 32):
        t = ints[:, :, b].astype(np.float32) * dw[None, :, b].astype(np.float32)
        t = (t * dx[:, None, b].astype(np.float32)).astype(np.float32)
        acc = (acc + t).astype(np.float32)
    assert O.q4_0_linear(x, blob, n).tobytes() == acc.tobytes()


@pytest.mark.parametrize("m", [2, 5, 17, 130])
@pytest.mark.parametrize("n", [8, 9, 10, 11])
def test_batched_rows_equal_one_row_calls_bit_for_bit(m, n):
    rng = np.random.default_rng(177 + m * 13 + n)
    k = 512
    blob = O.q4_0_quantize((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    x = (rng.standard_normal((m, k)) * 1.3).astype(np.float32)
    batched = O.q4_0_linear(x, blob, n, threads=3)
    rows = np.concatenate([O.q4_0_linear(x[i:i + 1], blob, n) for i in range(m)])
    assert batched.tobytes() == rows.tobytes()


def test_lossless_operands_give_the_exact_integer_matmul():
    rng = np.random.default_rng(1770)
    k = 64
    for n in (8, 9, 10, 11):
        nib = rng.integers(0, 16, size=(n, k // 32, 32))
        blob = bytearray()
        for r in range(n):
            for b in range(k // 32):
                blob += struct.pack("<e", 1.0) + bytes(int(nib[r, b, j] | (nib[r, b, j + 16] << 4)) for j in range(16))
        dense = (nib - 8).reshape(n, k)
        for m in (2, 5, 17, 130):
            xs = rng.integers(-126, 127, size=(m, k))
            xs[:, 0], xs[:, 32] = 127, -127
            got = O.q4_0_linear(xs.astype(np.float32), bytes(blob), n, threads=2)
            assert np.array_equal(got.astype(np.int64), xs @ dense.T)


def test_bias_is_added_after_the_matmul_in_float32():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 64)).astype(np.float32)
    blob = O.synth_q4_0_weight(6, 64, 0.02, 4)
    b = rng.standard_normal(6).astype(np.float32)
    assert O.q4_0_linear(x, blob, 6, bias=b).tobytes() == (O.q4_0_linear(x, blob, 6) + b).astype(np.float32).tobytes()


# --- q8_0 weights (K:652-757): the same recurrence with an int8 block dot ----


@pytest.mark.parametrize("rows,out_f,in_f,seed", [(1, 8, 64, 31), (3, 12, 512, 32), (2, 5, 1024, 33)])
def test_q8_0_linear_is_within_the_counted_bound_of_its_exact_value(rows, out_f, in_f, seed):
    w = (np.random.default_rng(seed + 1).standard_normal((out_f, in_f)) * 0.05).astype(np.float32)
    x = _tie_free(rows, in_f, seed)
    blob = O.q8_0_quantize(w)
    got = O.q8_0_linear(x, blob, out_f).astype(np.float64)
    exact, abs_sum, ref_err = O.exact_linear_q8_0(O.q8_0_quantize(x), blob, rows, out_f, in_f)
    bound = O.linear_bound(in_f, abs_sum, ref_err)
    assert np.max(np.abs(got - exact) / bound) <= 1.0
    # the bound refuses the matmul that skips activation quantisation
    wdq = O.q8_0_dequantize(blob, out_f * in_f).astype(np.float64).reshape(out_f, in_f)
    assert np.max(np.abs(x.astype(np.float64) @ wdq.T - exact) / bound) > 1.0


def test_q8_0_linear_matches_a_numpy_float32_restatement_bit_for_bit():
    """K:738-757 spelled in numpy float32: the int8 block dot, then the two
    roundings and the ordered sum; the q4_0 dot on the same bytes differs."""
    rng = np.random.default_rng(23)
    m, k, n = 3, 256, 40
    x = rng.standard_normal((m, k)).astype(np.float32)
    blob = O.synth_q8_0_weight(n, k, 0.02, 24)
    dw, qw = O.q8_0_parts(blob, n, k)
    dx, qx = O.q8_0_parts(O.q8_0_quantize(x), m, k)
    ints = np.einsum("rbk,obk->rob", qx, qw)
    acc = np.zeros((m, n), np.float32)
    for b in range(k // 32):
        t = ints[:, :, b].astype(np.float32) * dw[None, :, b].astype(np.float32)
        t = (t * dx[:, None, b].astype(np.float32)).astype(np.float32)
        acc = (acc + t).astype(np.float32)
    assert O.q8_0_linear(x, blob, n).tobytes() == acc.tobytes()
    xq = O.q8_0_quantize(x[0])
    assert O.vec_dot_q8_0_q8_0(k, blob[: (k // 32) * 34], xq) == float(acc[0, 0])


@pytest.mark.parametrize("m", [2, 5, 17, 130])
def test_q8_0_batched_rows_equal_one_row_calls_bit_for_bit(m):
    rng = np.random.default_rng(277 + m)
    k, n = 512, 11
    blob = O.q8_0_quantize((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    x = (rng.standard_normal((m, k)) * 1.3).astype(np.float32)
    batched = O.q8_0_linear(x, blob, n, threads=3)
    rows = np.concatenate([O.q8_0_linear(x[i:i + 1], blob, n) for i in range(m)])
    assert batched.tobytes() == rows.tobytes()


def test_q8_0_lossless_operands_give_the_exact_integer_matmul():
    """test_qgemm.py:103-137's q8_0 half: scale-1 blocks of integer codes and
    activation blocks with absmax 127 quantise exactly, so the result is the
    integer matmul."""
    rng = np.random.default_rng(1771)
    k = 64
    for n in (8, 9, 10, 11):
        codes = rng.integers(-127, 128, size=(n, k // 32, 32))
        blob = bytearray()
        for r in range(n):
            for b in range(k // 32):
                blob += struct.pack("<e", 1.0) + struct.pack("<32b", *codes[r, b])
        dense = codes.reshape(n, k)
        for m in (2, 5, 17, 130):
            xs = rng.integers(-126, 127, size=(m, k))
            xs[:, 0], xs[:, 32] = 127, -127
            got = O.q8_0_linear(xs.astype(np.float32), bytes(blob), n, threads=2)
            assert np.array_equal(got.astype(np.int64), xs @ dense.T)


# --- 4. planted faults fail the fixtures -------------------------------------


def _np_q4_0_quantize(x, *, unsigned_scale=False):
    x = np.asarray(x, np.float32).reshape(-1, 32)
    out = bytearray()
    for blk in x:
        i = int(np.argmax(np.abs(blk)))  # first index of the largest |x|
        mx = np.float32(np.abs(blk[i]) if unsigned_scale else blk[i])
        d = np.float32(mx / np.float32(-8.0))
        inv = np.float32(1.0) / d if d != 0 else np.float32(0.0)
        out += np.array([d], np.float32).astype(np.float16).tobytes()
        q = np.minimum(15, np.clip(np.trunc((blk * inv).astype(np.float32) + np.float32(8.5)), 0, 255)).astype(np.uint8)
        out += bytes((q[:16] | (q[16:] << 4)).astype(np.uint8))
    return bytes(out)


def _np_q8_0_quantize(x, *, half_even=False, f16_inverse=False):
    x = np.asarray(x, np.float32).reshape(-1, 32)
    out = bytearray()
    for blk in x:
        d = np.float32(np.max(np.abs(blk)) / np.float32(127.0))
        dd = np.float32(np.float16(d)) if f16_inverse else d
        inv = np.float32(1.0) / dd if dd != 0 else np.float32(0.0)
        v = (blk * inv).astype(np.float32)
        r = np.round(v) if half_even else np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))
        out += np.array([d], np.float32).astype(np.float16).tobytes()
        out += np.clip(r, -128, 127).astype(np.int8).tobytes()
    return bytes(out)


def test_planted_faults_are_caught_by_the_fixtures(golden):
    cases, _ = golden
    q4 = [c for (f, _), c in cases.items() if f == "q4_0" and "input_f32" in c]
    q8 = [c for (f, _), c in cases.items() if f == "q8_0" and "input_f32" in c]
    # the numpy restatement itself is right...
    for c in q4:
        assert _np_q4_0_quantize(_f32_list(c["input_f32"])) == bytes.fromhex(c["blob"])
    for c in q8:
        assert _np_q8_0_quantize(_f32_list(c["input_f32"])) == bytes.fromhex(c["blob"])
    # ...and each planted fault is caught by at least one case
    assert any(_np_q4_0_quantize(_f32_list(c["input_f32"]), unsigned_scale=True) != bytes.fromhex(c["blob"]) for c in q4)
    assert any(_np_q8_0_quantize(_f32_list(c["input_f32"]), half_even=True) != bytes.fromhex(c["blob"]) for c in q8)
    # a reader pairing nibbles (j, j+1) instead of (j, j+16)
    c = cases[("q4_0", "gauss")]
    blob = bytes.fromhex(c["blob"])
    d = np.frombuffer(blob[:2], np.float16).astype(np.float32)[0]
    qs = np.frombuffer(blob[2:18], np.uint8)
    wrong = np.empty(32, np.float32)
    wrong[0::2] = ((qs & 0xF).astype(np.int32) - 8).astype(np.float32) * d
    wrong[1::2] = ((qs >> 4).astype(np.int32) - 8).astype(np.float32) * d
    assert wrong.tobytes() != bytes.fromhex(c["dequant_f32"])
