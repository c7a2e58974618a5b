"""The oracle's dense linear (the checker of tn_dense_linear, the `format="f32"`
exactness control's matmul), pinned on the CPU by what the mathematics fixes:

- integer-valued operands small enough that every product and partial sum is
  an integer below 2^24: any summation order gives the exact integer sum,
  computed here with Python ints (the reference's own control test uses such
  operands, tests/_support/test_shim.py:13011-13061);
- random operands within the standard bound gamma_K * sum|x w| of the exact
  float64 value;
- the order itself, by known answers a different order or an unfused
  multiply-add gets wrong: x = (2^24, 1, -2^24) gives 0 in k order (the 1 is
  rounded away against 2^24) and 1 in reverse order; x = (-1, a), w = (1, a)
  with a = 1 + 2^-12 gives 2^-11 + 2^-24 with a fused chain and 2^-11 with
  the product rounded first;
- a transposed weight (a planted mistake) fails the integer check.
"""

import numpy as np

import oracle as O


def _ints(rows, cols, amax, seed):
    return np.random.default_rng(seed).integers(-amax, amax + 1, (rows, cols)).astype(np.float32)


def _exact(x, w, b=None):
    xi, wi = x.astype(np.int64), w.astype(np.int64)
    want = [[int(sum(int(a) * int(c) for a, c in zip(xr, wr))) for wr in wi] for xr in xi]
    out = np.array(want, dtype=np.float64)
    return out if b is None else out + b.astype(np.float64)[None, :]


def test_integer_operands_give_the_exact_sums():
    for k, n in ((32, 4), (64, 3), (256, 2), (17, 5)):
        w = _ints(n, k, 64, 100 + k)
        x = _ints(3, k, 64, 200 + k)
        b = np.arange(n, dtype=np.float32) - n // 2
        for bias in (None, b):
            got = O.dense_linear(x, w, bias)
            assert np.array_equal(got.astype(np.float64), _exact(x, w, bias)), (k, n, bias is not None)


def test_a_transposed_weight_is_caught():
    k, n = 32, 32
    w = _ints(n, k, 64, 7)
    x = _ints(3, k, 64, 8)
    assert not np.array_equal(O.dense_linear(x, w.T.copy()).astype(np.float64), _exact(x, w))


def test_random_operands_within_the_accumulation_bound():
    rng = np.random.default_rng(3)
    for m, k, n in ((1, 1, 1), (5, 576, 7), (9, 1536, 3)):
        x = rng.standard_normal((m, k)).astype(np.float32)
        w = rng.standard_normal((n, k)).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        got = O.dense_linear(x, w, b).astype(np.float64)
        prod = x.astype(np.float64) @ w.T.astype(np.float64)
        exact = prod + b.astype(np.float64)
        bound = O.gamma(k) * (np.abs(x.astype(np.float64)) @ np.abs(w.T.astype(np.float64)))
        bound = bound + 2.0 ** -24 * np.abs(exact) * 1.01  # the bias addition's rounding
        assert np.all(np.abs(got - exact) <= bound), (m, k, n)


def test_the_chain_runs_in_k_order():
    w = np.ones((1, 3), np.float32)
    fwd = np.array([[2.0 ** 24, 1.0, -(2.0 ** 24)]], np.float32)
    assert O.dense_linear(fwd, w)[0, 0] == 0.0
    assert O.dense_linear(fwd[:, ::-1].copy(), w)[0, 0] == 1.0


def test_the_chain_fuses_each_multiply_add():
    a = np.float32(1.0 + 2.0 ** -12)
    x = np.array([[-1.0, a]], np.float32)
    w = np.array([[1.0, a]], np.float32)
    assert O.dense_linear(x, w)[0, 0] == np.float32(2.0 ** -11 + 2.0 ** -24)
    # the unfused value, for contrast: the product rounds to 1 + 2^-11 first
    assert np.float32(np.float32(a * a) - np.float32(1.0)) == np.float32(2.0 ** -11)


def test_batched_rows_equal_one_row_calls():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 100)).astype(np.float32)
    w = rng.standard_normal((9, 100)).astype(np.float32)
    full = O.dense_linear(x, w)
    for i in range(6):
        assert np.array_equal(O.dense_linear(x[i:i + 1], w)[0], full[i])
