"""The SDPA tolerance is a formula, not a free parameter: pin its terms."""

import numpy as np

import oracle as O


def test_tolerance_terms_are_the_stated_formula():
    r64 = np.array([1.5, -0.25, 3.0])
    r32 = r64 + np.array([1e-7, 0.0, -2e-7])
    t = O.sdpa_tolerance(r32, r64)
    assert np.allclose(t, max(4 * 2e-7, 1.186e-6 * 3.0))
    tb = O.sdpa_tolerance(r32, r64, "bfloat16", p=np.array([1.0, 1.0, 1.0]))
    # + one bf16 ulp at the value's binade + 2^-8 * sum P|V|
    assert np.allclose(tb - t, np.array([2.0 ** -7, 2.0 ** -9, 2.0 ** -6]) + 2.0 ** -8)
    # spacing taken at the larger of |ref| and |got|
    tg = O.sdpa_tolerance(r32, r64, "bfloat16", got=np.array([2.0, 0.0, 0.0]))
    assert np.isclose(tg[0] - t[0], 2.0 ** -6)


def test_bf16_unit_roundoff_is_two_to_minus_eight():
    rng = np.random.default_rng(0)
    x = rng.uniform(1, 2, 100000).astype(np.float32)
    r = O.bf16_to_f32(O.bf16_from_f32(x))
    assert np.max(np.abs(r - x) / x) <= 2.0 ** -8
    assert np.max(np.abs(r - x) / x) > 2.0 ** -9  # and 2^-9 would be too small


def test_f16_terms_ulp_subnormal_spacing_and_underflow():
    r64 = np.array([1.5, -0.25, 3.0, 1e-6])
    r32 = r64.copy()
    t = O.sdpa_tolerance(r32, r64)
    th = O.sdpa_tolerance(r32, r64, "float16", p=np.ones(4), vsum=np.full(4, 2.0))
    # one f16 ulp at the binade (at 1e-6, below 2^-14, the subnormal spacing
    # 2^-24), 2^-11 * sum P|V|, 2^-25 * sum |V|
    ulp = np.array([2.0 ** -10, 2.0 ** -12, 2.0 ** -9, 2.0 ** -24])
    assert np.allclose(th - t, ulp + 2.0 ** -11 + 2.0 ** -24)


def test_f16_rounding_error_is_within_the_stated_terms():
    """numpy's float16 rounding (the oracle's f16 narrowing) stays within half
    the stated spacing, down into the subnormals; a probability rounded to f16
    is off by at most 2^-11 of itself or 2^-25."""
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(1, 2, 50000), 2.0 ** rng.uniform(-30, -14, 50000)]).astype(np.float32)
    r = x.astype(np.float16).astype(np.float32).astype(np.float64)
    err = np.abs(r - x)
    assert np.all(err <= np.maximum(2.0 ** -11 * x, 2.0 ** -25))
    # halving either term fails somewhere
    assert np.any(err > np.maximum(2.0 ** -12 * x, 2.0 ** -25))
    assert np.any(err > np.maximum(2.0 ** -11 * x, 2.0 ** -26))
