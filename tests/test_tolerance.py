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
