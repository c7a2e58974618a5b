"""The oracle's decode-step restatement (oracle/decoder.py), pinned by what
the mathematics fixes rather than by retyping its formulas: rotation
identities for RoPE, the odd-part identity of SiLU, closed forms and scale
invariance for RMSNorm, argmax's documented tie and NaN rules, a one-key
attention, and the float32 run's agreement with the float64 one."""

import numpy as np
import pytest

import oracle as O
from oracle import decoder as OD

CFG = OD.LlamaConfig()


def test_inv_freq_is_one_over_theta_to_the_2i_over_d():
    f = OD.inv_freq(CFG)
    assert f.dtype == np.float32 and f.shape == (32,)
    assert f[0] == 1.0
    exact = 1.0 / (1e5 ** (np.arange(0, 64, 2) / 64.0))
    assert np.max(np.abs(f - exact) / exact) < 4e-7  # float32 rounding of pow and of the division


def test_rope_is_a_rotation_by_pos_times_the_frequency():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 64))
    f = OD.inv_freq(CFG).astype(np.float64)
    assert np.array_equal(OD.rope(x, 0, f, np.float64), x)  # position 0
    for pos in (1, 17, 300):
        y = OD.rope(x, pos, f, np.float64)
        # the complex-number form: (x1 + i x2) * exp(i pos f)
        z = (x[:, :32] + 1j * x[:, 32:]) * np.exp(1j * pos * f)
        assert np.allclose(y[:, :32], z.real, rtol=0, atol=1e-12)
        assert np.allclose(y[:, 32:], z.imag, rtol=0, atol=1e-12)
        # pairs keep their length, and rotations compose
        assert np.allclose(np.hypot(y[:, :32], y[:, 32:]), np.hypot(x[:, :32], x[:, 32:]), atol=1e-12)
        assert np.allclose(OD.rope(OD.rope(x, 5, f, np.float64), pos, f, np.float64),
                           OD.rope(x, 5 + pos, f, np.float64), atol=1e-11)


def test_silu_odd_part_identity():
    x = np.linspace(-20, 20, 4001)
    one = np.ones_like(x)
    s = OD.silu_mul(x, one, np.float64)
    # x * sigmoid(x) - (-x) * sigmoid(-x) = x, and silu(0) = 0
    assert np.allclose(s - OD.silu_mul(-x, one, np.float64), x, atol=1e-12)
    assert OD.silu_mul(np.array([0.0]), np.array([1.0]), np.float64)[0] == 0.0


def test_rmsnorm_closed_form_and_scale_invariance():
    c = 3.0
    y = OD.rmsnorm(np.full(576, c), np.ones(576), 1e-5, np.float64)
    assert np.allclose(y, c / np.sqrt(c * c + 1e-5), rtol=1e-15)
    rng = np.random.default_rng(2)
    x = rng.standard_normal(576).astype(np.float32)
    w = rng.standard_normal(576).astype(np.float32)
    # eps = 0: scaling the row by a power of two changes no bit
    assert np.array_equal(OD.rmsnorm(x, w, 0.0), OD.rmsnorm(x * np.float32(8), w, 0.0))
    # and the weight multiplies the normalised row
    assert np.array_equal(OD.rmsnorm(x, w, 1e-5), w * OD.rmsnorm(x, np.ones(576, np.float32), 1e-5))


def test_argmax_rules():
    assert OD.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert OD.argmax([-np.inf, -np.inf]) == 0
    assert OD.argmax([1.0, np.nan, np.inf, np.nan]) == 1


def test_one_key_attention_returns_v():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 9, 1, 64)).astype(np.float32)
    k = rng.standard_normal((1, 3, 1, 64)).astype(np.float32)
    v = rng.standard_normal((1, 3, 1, 64)).astype(np.float32)
    out, _ = O.sdpa(q, k, v)
    assert np.array_equal(out[0, :, 0], np.repeat(v[0, :, 0], 3, axis=0))


SMALL = OD.LlamaConfig(n_layers=2, hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, inter=256, vocab=512)


def test_decoder_float32_run_tracks_the_float64_run():
    r32 = OD.Decoder(SMALL, 3, 8, np.float32)
    r64 = OD.Decoder(SMALL, 3, 8, np.float64)
    for pos, tok in enumerate([7, 300, 2, 511]):
        a, b = r32.step(tok, pos), r64.step(tok, pos)
        assert a.dtype == np.float32 and a.shape == (SMALL.vocab,)
        assert np.max(np.abs(a - b)) < 1e-3 * np.max(np.abs(b)), pos


def test_stacked_projections_equal_separate_ones():
    """Stacking q|k|v (and gate|up) row-wise changes no bit of the quantised
    linear: each output row is its own recurrence."""
    w = OD.layer_weights(SMALL, 0, 4)
    x = np.random.default_rng(5).standard_normal((1, SMALL.hidden)).astype(np.float32)
    blob = O.q4_0_quantize(w["qkv"])
    full = O.q4_0_linear(x, blob, w["qkv"].shape[0])
    q = w["qkv"][:128]
    assert np.array_equal(full[:, :128], O.q4_0_linear(x, O.q4_0_quantize(q), 128))


@pytest.mark.parametrize("n", [1, 5])
def test_model_weights_are_deterministic(n):
    a = OD.layer_weights(SMALL, n, 9)
    b = OD.layer_weights(SMALL, n, 9)
    assert all(np.array_equal(a[k], b[k]) for k in a)
    c = OD.layer_weights(SMALL, n, 10)
    assert not np.array_equal(a["qkv"], c["qkv"])


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_a_whole_sequence_at_once_equals_step_by_step(dtype):
    """The batched teacher-forced run (used to check the full-size model)
    gives step()'s logits: row-wise ops are row-wise and the attention of row
    t sees keys 0..t. float32: within a few ulp-sized steps of the logits'
    scale (the batched C attention sums in the same order, and the q4 linear
    is row-independent bit for bit); float64 likewise."""
    cfg = OD.LlamaConfig(n_layers=2, hidden=128, n_heads=6, n_kv_heads=2, head_dim=64, inter=256, vocab=512)
    toks = [3, 500, 17, 17, 0, 256, 99, 1, 2, 77, 300, 411]
    dec = OD.Decoder(cfg, 5, 16, dtype)
    want = {p: dec.step(t, p) for p, t in enumerate(toks)}
    got = OD.teacher_forced_logits(OD.Decoder(cfg, 5, 16, dtype), toks, range(len(toks)))
    for p in range(len(toks)):
        scale = float(np.max(np.abs(want[p])))
        rel = 1e-5 if dtype == np.float32 else 1e-12
        assert float(np.max(np.abs(got[p] - want[p]))) <= rel * scale


def test_the_float64_linear_rows_is_the_exact_quantised_product():
    """linear_rows in float64 against the exact dyadic value of the same
    quantised product (exact_linear_q4_0) within its rounding bound."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 96)).astype(np.float32)
    w = (rng.standard_normal((40, 96)) * 0.02).astype(np.float32)
    blob = O.q4_0_quantize(w)
    got = OD.linear_rows(x, blob, 40, np.float64)
    value, abs_sum, ref_err = O.exact_linear_q4_0(O.q8_0_quantize(x), blob, 5, 40, 96)
    assert np.all(np.abs(got - value) <= ref_err + 96 * 2.0 ** -53 * abs_sum)
    # and the float32 rows are the C oracle's one-row calls, bit for bit
    f32 = OD.linear_rows(x, blob, 40, np.float32, threads=3)
    assert all(np.array_equal(f32[i], O.q4_0_linear(x[i:i + 1], blob, 40)[0]) for i in range(5))


# ---- the composition, pinned by models whose answer the mathematics fixes ----
#
# The checks above pin each op; these pin how the decoder puts them together
# (pre-norm, the residual stream, the final norm and lm_head, the causal
# extent of the attention and its GQA head map) with weights that make the
# answer known in closed form. A zero q4_0 weight quantises to zero scales, so
# its linear is exactly 0 for any input.
GQA = OD.LlamaConfig(n_layers=3, hidden=384, n_heads=6, n_kv_heads=2, head_dim=64, inter=256, vocab=512)


def _zeroed(cfg, seed, *, qk=False, o_down=False):
    """cfg's seeded weights with the q and k rows of every qkv projection, or
    every o and down projection, set to zero."""
    D = cfg.head_dim
    layers = []
    for i in range(cfg.n_layers):
        w = dict(OD.layer_weights(cfg, i, seed))
        if qk:
            w["qkv"] = w["qkv"].copy()
            w["qkv"][:(cfg.n_heads + cfg.n_kv_heads) * D] = 0.0
        if o_down:
            w["o"] = np.zeros_like(w["o"])
            w["down"] = np.zeros_like(w["down"])
        layers.append(w)
    return layers, OD.model_weights(cfg, seed)


def test_zero_weight_linear_is_exactly_zero():
    x = np.random.default_rng(0).standard_normal((3, 96)).astype(np.float32)
    blob = O.q4_0_quantize(np.zeros((40, 96), np.float32))
    assert np.array_equal(O.q4_0_linear(x, blob, 40), np.zeros((3, 40), np.float32))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_without_o_and_down_the_logits_are_lm_head_of_the_normed_embedding(dtype):
    """With every o and down projection zero, each layer adds exact zeros to
    the residual stream, so at every position h is the token's embedding row
    and the logits are lm_head(rmsnorm(embed[t], norm)): this pins that the
    layers add to the residual stream (not to a normed copy), that nothing
    else is added, and the final norm and lm_head."""
    layers, top = _zeroed(GQA, 7, o_down=True)
    toks = [5, 400, 5, 17, 256, 0, 511, 99]
    dec = OD.Decoder(GQA, 7, 16, dtype, layers, top)
    batched = OD.teacher_forced_logits(OD.Decoder(GQA, 7, 16, dtype, layers, top), toks, range(len(toks)))
    for p, t in enumerate(toks):
        x = OD.rmsnorm(top["embed"][t].astype(dtype), top["norm"], GQA.eps, dtype)
        want = OD.linear(x, dec.lm_blob, GQA.vocab, dtype).astype(dtype)
        assert np.array_equal(dec.step(t, p), want), p
        assert np.array_equal(batched[p], want), p


@pytest.mark.parametrize("batched", [False, True])
def test_with_q_and_k_zero_each_head_attends_uniformly_to_keys_0_to_t(batched):
    """With the q and k rows zero, every score is 0, so the attention of the
    row at position t is the plain mean of the value rows 0..t of its key/value
    head h // (Hq / Hkv): this pins the causal extent (position t itself
    included, nothing after it) and the GQA head map, in every layer, for the
    step and the whole-sequence run. float64, so the mean is compared at
    1e-13 of the values' scale."""
    layers, top = _zeroed(GQA, 8, qk=True)
    toks = [3, 3, 450, 12, 77, 0, 300, 511, 2, 2, 64]
    T, Hq, Hkv, D = len(toks), GQA.n_heads, GQA.n_kv_heads, GQA.head_dim
    rep = Hq // Hkv
    if batched:
        trace = []
        OD.teacher_forced_logits(OD.Decoder(GQA, 8, 16, np.float64, layers, top), toks, [T - 1], trace=trace)
        per_layer = [(tr["a"], tr["v"]) for tr in trace]  # a [T, Hq*D], v [T, Hkv, D]
    else:
        dec = OD.Decoder(GQA, 8, 16, np.float64, layers, top)
        steps = []
        for p, t in enumerate(toks):
            tr = []
            dec.step(t, p, trace=tr)
            steps.append(tr)
        per_layer = []
        for li in range(GQA.n_layers):
            a = np.stack([steps[p][li]["a"] for p in range(T)])
            v = steps[-1][li]["v"].transpose(1, 0, 2)  # the full cache after the last step [T, Hkv, D]
            # the cache rows a step read are the rows the last step sees (no row is rewritten)
            for p in range(T):
                assert np.array_equal(steps[p][li]["v"], steps[-1][li]["v"][:, :p + 1])
            per_layer.append((a, v))
    assert len(per_layer) == GQA.n_layers
    for a, v in per_layer:
        a = a.reshape(T, Hq, D)
        scale = float(np.max(np.abs(v)))
        for t in range(T):
            for h in range(Hq):
                want = v[:t + 1, h // rep].mean(axis=0)
                assert np.max(np.abs(a[t, h] - want)) <= 1e-13 * scale, (t, h)
        # and the map is not the identity or a modulo: heads of different kv heads differ
        assert not np.allclose(a[:, 0], a[:, rep])
