"""Seeded random shapes through the hot path on the MI355X, against the CPU
oracle with the same bars as the focused tests: SDPA prefill and decode
within the derived bound (test_sdpa_gpu's checks), the q4_0 / q8_0 / q4_k
linears bit for bit. The shapes are drawn once, at collection, from a fixed
seed: odd lengths, q_len above and below kv_len, every GQA ratio the kernels
take, head dims on the MFMA kernels and on the plain one, empty and
truncated decode sequences, GEMV and GEMM row counts, rows of one block and
long rows, and bool masks broadcast from each shape the kernels read in
place. Each case is sized so that the oracle finishes in a second or so.
"""

import numpy as np
import pytest

import oracle as O
from test_sdpa_gpu import _check, _decode_case, _det
from test_sdpa_mask_gpu import _bool_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


def _prefill_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        b = int(rng.integers(1, 3))
        hkv = int(rng.choice([1, 2]))
        hq = hkv * int(rng.choice([1, 2, 3, 4, 8]))
        d = int(rng.choice([64, 64, 128, 128, 32, 80]))
        l = int(rng.integers(1, 300))
        s = int(rng.integers(1, 700))
        causal = bool(rng.integers(0, 2))
        dtype = str(rng.choice(["float32", "bfloat16", "float16"]))
        if b * hq * l * s * d > 80_000_000:
            continue
        out.append((b, hq, hkv, l, s, d, causal, dtype))
    return out


def _decode_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        b = int(rng.integers(1, 40))
        hkv = int(rng.choice([1, 2, 4]))
        hq = hkv * int(rng.choice([1, 2, 3, 4, 8]))
        d = int(rng.choice([64, 128]))
        cap = int(rng.integers(1, 700))
        lens = [int(x) for x in rng.integers(0, cap + 1, size=b)]
        dtype = str(rng.choice(["bfloat16", "float16", "float32"]))
        if b * hq * cap * d > 30_000_000:
            continue
        out.append((b, hq, hkv, d, cap, lens, dtype))
    return out


def _linear_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        fmt = ["q4_0", "q8_0", "q4_k"][i % 3]
        m = int(rng.choice([1, 2, 3, 4, 5, 9, 33]))
        nn = int(rng.integers(1, 400))
        k = 256 * int(rng.integers(1, 9)) if fmt == "q4_k" else 32 * int(rng.integers(1, 65))
        out.append((fmt, m, nn, k, int(rng.integers(0, 1 << 30))))
    return out


def _mask_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        b = int(rng.integers(1, 3))
        hkv = int(rng.choice([1, 2]))
        hq = hkv * int(rng.choice([1, 2, 3, 4]))
        d = int(rng.choice([64, 128, 80]))
        l = int(rng.integers(1, 160))
        s = int(rng.integers(1, 300))
        shape = str(rng.choice(["full", "LS", "B1LS", "B11S"]))
        density = float(rng.uniform(0.3, 0.95))
        dtype = str(rng.choice(["float32", "bfloat16", "float16"]))
        if b * hq * l * s * d > 40_000_000:
            continue
        out.append((b, hq, hkv, l, s, d, shape, density, dtype, int(rng.integers(0, 1 << 30))))
    return out


PREFILL = _prefill_cases(48, 2026)
DECODE = _decode_cases(24, 2027)
LINEAR = _linear_cases(36, 2028)
MASKED = _mask_cases(24, 2029)


@pytest.mark.parametrize("case", PREFILL, ids=[f"p{i}" for i in range(len(PREFILL))])
def test_prefill_sweep(tn, case):
    b, hq, hkv, l, s, d, causal, dtype = case
    print("case", case, flush=True)
    q, k, v = _det((b, hq, l, d), 1), _det((b, hkv, s, d), 2), _det((b, hkv, s, d), 3)
    _check(tn, dtype, q, k, v, causal)


@pytest.mark.parametrize("case", DECODE, ids=[f"d{i}" for i in range(len(DECODE))])
def test_decode_sweep(tn, case):
    b, hq, hkv, d, cap, lens, dtype = case
    print("case", (b, hq, hkv, d, cap, dtype), flush=True)
    _decode_case(tn, b, hq, hkv, d, lens, cap, seed=b * 31 + cap, dtype=dtype)


@pytest.mark.parametrize("case", LINEAR, ids=[f"l{i}" for i in range(len(LINEAR))])
def test_linear_sweep(tn, case):
    fmt, m, n, k, seed = case
    print("case", case, flush=True)
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32) if seed % 2 else None
    if fmt == "q4_0":
        blob = O.synth_q4_0_weight(n, k, 0.02, seed % 1000)
        want = O.q4_0_linear(x, blob, n, bias=bias, threads=8)
    elif fmt == "q8_0":
        blob = O.synth_q8_0_weight(n, k, 0.02, seed % 1000)
        want = O.q8_0_linear(x, blob, n, bias=bias, threads=8)
    else:
        blob = O.synth_q4_k_weight(n, k, seed % 1000)
        want = O.q4_k_linear(x, blob, n, bias=bias, threads=8)
    q = tn._quantized_from_blob(blob, (n, k), fmt, device="hip")
    bb = tn.tensor(bias, device="hip") if bias is not None else None
    got = tn._quantized_linear(tn.tensor(x, device="hip"), q, bb).numpy()
    assert got.tobytes() == want.tobytes(), np.argwhere(got != want)[:5]


@pytest.mark.parametrize("case", MASKED, ids=[f"m{i}" for i in range(len(MASKED))])
def test_bool_mask_sweep(tn, case):
    """F.sdpa with a random bool mask, broadcast by strides from its own
    shape; rows the mask hides entirely must come out NaN."""
    b, hq, hkv, l, s, d, shape, density, dtype, seed = case
    print("case", case, flush=True)
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal(sh) for sh in ((b, hq, l, d), (b, hkv, s, d), (b, hkv, s, d)))
    mshape = {"full": (b, hq, l, s), "LS": (l, s), "B1LS": (b, 1, l, s), "B11S": (b, 1, 1, s)}[shape]
    mask = rng.random(mshape) < density
    full = np.broadcast_to(mask, (b, hq, l, s))
    nan_rows = [tuple(int(x) for x in r) for r in np.argwhere(~full.any(axis=-1))]
    _bool_case(tn, dtype, q, k, v, mask, nan_rows=nan_rows)
