"""Pins the CPU oracle's SDPA (the reference's default path, aten.rs:10330-10423).

* The fp64 restatement against an fp64 closed form written independently in
  numpy (explicit repeat_interleave of kv heads, explicit upper-left tril mask).
* Special cases the mathematics fixes: upper-left causal with L != S (row t
  keeps keys 0..=t, aten.rs:10038-10041), the GQA head map i -> i / n_rep
  (aten.rs:17074-17081; tiling i % n_rep must fail), the default scale, the
  logsumexp over masked+scaled scores, a single key (softmax == 1), identical
  keys (uniform weights -> mean of V).
* The fp32 restatement against fp64 within the derived tolerance, on the
  reference's own test shapes (tests/_support/test_shim.py:12075-12083) with
  its exactly-representable inputs (:12103-12116).
* The third-party upstream torch CPU op (installed here; the reference's
  default path agrees with it to 1e-6 in fp32, test_shim.py:12415-12440),
  checked at the same bound.
"""

import math

import numpy as np
import pytest

import oracle as O

SDPA_SHAPES = [
    # (batch, query heads, kv heads, q_len, kv_len, head_dim)
    (1, 2, 2, 8, 8, 16),
    (1, 9, 3, 26, 26, 64),
    (1, 2, 2, 33, 33, 8),
    (1, 2, 2, 70, 70, 8),
    (1, 1, 1, 40, 600, 8),
    (1, 1, 1, 2, 5, 4),
]


def _det(shape, seed):
    n = int(np.prod(shape))
    return np.array(O.sdpa_det(n, seed), dtype=np.float64).reshape(shape)


def _inputs(shape):
    b, hq, hkv, l, s, d = shape
    return _det((b, hq, l, d), 1), _det((b, hkv, s, d), 2), _det((b, hkv, s, d), 3)


@pytest.mark.parametrize("shape", SDPA_SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_fp64_restatement_matches_the_closed_form(shape, causal):
    q, k, v = _inputs(shape)
    out, lse = O.sdpa(q, k, v, is_causal=causal, dtype=np.float64)
    want_o, want_l = O.sdpa_closed_form(q, k, v, is_causal=causal)
    assert np.max(np.abs(out - want_o)) <= 1e-13 * max(1.0, np.max(np.abs(want_o)))
    assert np.max(np.abs(lse - want_l)) <= 1e-13 * max(1.0, np.max(np.abs(want_l)))


def test_causal_is_upper_left_when_l_differs_from_s():
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 1, 2, 4))
    k = rng.standard_normal((1, 1, 5, 4))
    v = rng.standard_normal((1, 1, 5, 4))
    out, _ = O.sdpa(q, k, v, is_causal=True, dtype=np.float64)
    # row 0 sees key 0 only -> exactly v[0]; row 1 sees keys 0..1
    assert np.allclose(out[0, 0, 0], v[0, 0, 0], rtol=0, atol=1e-15)
    s = q[0, 0, 1] @ k[0, 0, :2].T / 2.0
    p = np.exp(s - s.max()) / np.exp(s - s.max()).sum()
    assert np.allclose(out[0, 0, 1], p @ v[0, 0, :2], rtol=0, atol=1e-14)
    # the bottom-right reading differs on every element
    br = np.triu(np.ones((2, 5), bool), k=5 - 2 + 1)
    wrong, _ = O.sdpa_closed_form(q, k, v, mask=np.where(br, -np.inf, 0.0))
    assert np.all(np.abs(wrong - out) > 1e-6)


def test_gqa_maps_query_head_i_to_kv_head_i_over_n_rep():
    q, k, v = _inputs((1, 9, 3, 6, 6, 8))
    out, _ = O.sdpa(q, k, v, dtype=np.float64)
    for h in range(9):
        one, _ = O.sdpa(q[:, h:h + 1], k[:, h // 3:h // 3 + 1], v[:, h // 3:h // 3 + 1], dtype=np.float64)
        assert np.array_equal(one[:, 0], out[:, h])
    tiled, _ = O.sdpa(q[:, 1:2], k[:, 1 % 3:1 % 3 + 1], v[:, 1:2], dtype=np.float64)
    assert not np.allclose(tiled[:, 0], out[:, 1])


def test_single_key_and_identical_keys():
    rng = np.random.default_rng(9)
    q = rng.standard_normal((1, 2, 3, 8))
    k = rng.standard_normal((1, 2, 1, 8))
    v = rng.standard_normal((1, 2, 1, 8))
    out, lse = O.sdpa(q, k, v, dtype=np.float64)
    assert np.array_equal(out, np.broadcast_to(v, out.shape))
    assert np.allclose(lse, np.einsum("bhld,bhsd->bhl", q, k) / math.sqrt(8), rtol=0, atol=1e-15)
    k4 = np.repeat(k, 4, axis=2)
    v4 = rng.standard_normal((1, 2, 4, 8))
    out4, lse4 = O.sdpa(q, k4, v4, dtype=np.float64)
    assert np.allclose(out4, v4.mean(axis=2, keepdims=True).repeat(3, axis=2), rtol=0, atol=1e-15)
    assert np.allclose(lse4, lse + math.log(4), rtol=0, atol=1e-14)


def test_mask_is_added_after_scaling_and_fully_masked_rows_are_nan():
    rng = np.random.default_rng(10)
    q = rng.standard_normal((1, 1, 3, 4))
    k = rng.standard_normal((1, 1, 5, 4))
    v = rng.standard_normal((1, 1, 5, 4))
    mask = rng.standard_normal((1, 1, 3, 5))
    mask[0, 0, 2, :] = -np.inf
    out, lse = O.sdpa(q, k, v, mask=mask, dtype=np.float64)
    with np.errstate(invalid="ignore"):
        want, wl = O.sdpa_closed_form(q, k, v, mask=mask)
    assert np.allclose(out[0, 0, :2], want[0, 0, :2], rtol=0, atol=1e-14)
    # the default path shifts by the row maximum: -inf - -inf is NaN (aten.rs:10392-10395)
    assert np.all(np.isnan(out[0, 0, 2])) and np.isnan(lse[0, 0, 2])


@pytest.mark.parametrize("shape", SDPA_SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_fp32_restatement_is_within_the_derived_tolerance(shape, causal):
    q, k, v = _inputs(shape)
    o32, l32 = O.sdpa(q, k, v, is_causal=causal)
    o64, l64 = O.sdpa(q, k, v, is_causal=causal, dtype=np.float64)
    # the fp32 restatement's own error sets the tolerance, so here the check is
    # that this error is of float32 size: within 1e-6 (test_shim.py:12427) of
    # the tensor's scale (the lse of a 600-key row is ~6.5, where 1e-6 is 2 ulp)
    assert np.max(np.abs(o32 - o64)) <= 1e-6 * max(1.0, np.max(np.abs(o64)))
    assert np.max(np.abs(l32 - l64)) <= 1e-6 * max(1.0, np.max(np.abs(l64)))


def test_bf16_inputs_are_widened_and_the_output_narrowed_rne():
    q, k, v = _inputs((1, 2, 2, 8, 8, 16))
    qb, kb, vb = (O.bf16_from_f32(a.astype(np.float32)) for a in (q, k, v))
    ob, lb = O.sdpa_bf16(qb, kb, vb, is_causal=True)
    o32, l32 = O.sdpa(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), is_causal=True)
    assert np.array_equal(ob, O.bf16_from_f32(o32))
    assert np.array_equal(lb, l32)


def test_against_upstream_torch_cpu_op():
    torch = pytest.importorskip("torch")
    op = torch.ops.aten._scaled_dot_product_flash_attention_for_cpu
    worst = 0.0
    for shape in SDPA_SHAPES:
        b, hq, hkv, l, s, d = shape
        q, k, v = _inputs(shape)
        rep = hq // hkv
        for causal in (False, True):
            o32, l32 = O.sdpa(q, k, v, is_causal=causal)
            tq = torch.tensor(q, dtype=torch.float32)
            tk = torch.tensor(np.repeat(k, rep, axis=1), dtype=torch.float32)
            tv = torch.tensor(np.repeat(v, rep, axis=1), dtype=torch.float32)
            to, tl = op(tq, tk, tv, 0.0, causal)
            worst = max(worst, float(np.max(np.abs(to.numpy() - o32))), float(np.max(np.abs(tl.numpy() - l32))))
    assert worst <= 1e-6, worst
