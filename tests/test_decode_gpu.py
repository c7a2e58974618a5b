"""The decode-step ops and the q4_0 Llama decode step on the MI355X, against
the CPU oracle (oracle/decoder.py).

Bitwise where the op is exact or fully ordered (embedding gather, add,
argmax, KV append, the q4 linears inside the step). Elsewhere the bound is
the one used for SDPA: per tensor, 4x the oracle's own float32-vs-float64
distance on the same inputs, floored at 1.186e-6 of the tensor's scale
(oracle.sdpa_tolerance). The GPU sums the RMSNorm row as a tree and computes
cos/sin/exp with the device's libm, so these differ from the oracle's float32
run in the last bits only.
"""

import ctypes

import numpy as np
import pytest

import oracle as O
from oracle import decoder as OD

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


def _dev(tn, a, dtype=None):
    """A device copy. Bind it to a name for as long as a queued kernel reads
    it: a temporary's buffer is freed as soon as its last reference goes."""
    return tn.tensor(a, dtype=dtype, device="hip")


def _lib():
    from torchnative_amd import _lib

    return _lib


def _within(got, r32, r64):
    tol = O.sdpa_tolerance(r32, r64, "float32")
    worst = float(np.max(np.abs(np.asarray(got, np.float64) - r32) / tol))
    assert worst <= 1.0, f"{worst:.3g}x the bound"
    return worst


def test_embedding_gathers_rows_and_marks_bad_ids(tn):
    L = _lib()
    rng = np.random.default_rng(1)
    table = rng.standard_normal((50, 96)).astype(np.float32)
    ids = np.array([3, 0, 49, 7, -1, 50], np.int32)
    out = tn.empty((6, 96), "float32", "hip")
    d_ids, d_table = _dev(tn, ids), _dev(tn, table)
    L.check(L.lib().tn_embedding(None, d_ids.data_ptr(), 6, d_table.data_ptr(), 50, 96, out.data_ptr()))
    got = out.numpy()
    assert np.array_equal(got[:4], table[ids[:4]])
    assert np.all(np.isnan(got[4:]))


@pytest.mark.parametrize("m,n", [(1, 576), (3, 1536), (2, 100)])
def test_rmsnorm_within_the_derived_bound(tn, m, n):
    L = _lib()
    rng = np.random.default_rng(m * 1000 + n)
    x = rng.standard_normal((m, n)).astype(np.float32) * 3
    w = rng.standard_normal(n).astype(np.float32)
    y = tn.empty((m, n), "float32", "hip")
    d_x, d_w = _dev(tn, x), _dev(tn, w)
    L.check(L.lib().tn_rmsnorm(None, d_x.data_ptr(), m, n, d_w.data_ptr(), 1e-5, y.data_ptr()))
    _within(y.numpy(), OD.rmsnorm(x, w, 1e-5, np.float32).astype(np.float64),
            OD.rmsnorm(x.astype(np.float64), w, 1e-5, np.float64))
    # in place
    xd = _dev(tn, x)
    L.check(L.lib().tn_rmsnorm(None, xd.data_ptr(), m, n, d_w.data_ptr(), 1e-5, xd.data_ptr()))
    assert np.array_equal(xd.numpy(), y.numpy())


def test_rope_within_the_derived_bound(tn):
    L = _lib()
    cfg = OD.LlamaConfig()
    freqs = OD.inv_freq(cfg)
    rng = np.random.default_rng(3)
    pos = np.array([0, 1, 17, 255, 4000], np.int32)
    x = rng.standard_normal((5, 12, 64)).astype(np.float32)
    xd, d_f, d_p = _dev(tn, x), _dev(tn, freqs), _dev(tn, pos)
    L.check(L.lib().tn_rope(None, xd.data_ptr(), 5, 12, 64, d_f.data_ptr(), d_p.data_ptr()))
    got = xd.numpy()
    assert np.array_equal(got[0], x[0])  # position 0 is the identity: cos 0 = 1, sin 0 = 0
    for t in range(5):
        r32 = OD.rope(x[t], int(pos[t]), freqs, np.float32).astype(np.float64)
        r64 = OD.rope(x[t].astype(np.float64), int(pos[t]), freqs.astype(np.float64), np.float64)
        _within(got[t], r32, r64)


def test_silu_mul_and_add(tn):
    L = _lib()
    rng = np.random.default_rng(4)
    g = rng.standard_normal(3000).astype(np.float32) * 4
    u = rng.standard_normal(3000).astype(np.float32)
    out = tn.empty((3000,), "float32", "hip")
    d_g, d_u = _dev(tn, g), _dev(tn, u)
    L.check(L.lib().tn_silu_mul(None, d_g.data_ptr(), d_u.data_ptr(), 3000, out.data_ptr()))
    _within(out.numpy(), OD.silu_mul(g, u, np.float32).astype(np.float64),
            OD.silu_mul(g.astype(np.float64), u, np.float64))
    L.check(L.lib().tn_add(None, d_g.data_ptr(), d_u.data_ptr(), 3000, out.data_ptr()))
    assert np.array_equal(out.numpy(), g + u)


def test_argmax_first_max_and_nan(tn):
    L = _lib()
    rows = np.full((4, 5000), -1.0, np.float32)
    rows[0, [10, 4000, 4999]] = 7.0                 # ties: the first index
    rows[1, :] = -np.inf                            # all -inf: index 0
    rows[2, [3, 2000]] = np.nan                     # a NaN wins, the first one
    rows[2, 100] = np.inf
    rows[3] = np.random.default_rng(5).standard_normal(5000).astype(np.float32)
    out = tn.empty((4,), "int32", "hip")
    d_rows = _dev(tn, rows)
    L.check(L.lib().tn_argmax(None, d_rows.data_ptr(), 4, 5000, out.data_ptr()))
    assert out.numpy().tolist() == [OD.argmax(r) for r in rows] == [10, 0, 3, int(np.argmax(rows[3]))]


def test_kv_append_writes_at_the_device_position(tn):
    L = _lib()
    rng = np.random.default_rng(6)
    k = rng.standard_normal((2, 3, 64)).astype(np.float32)
    v = rng.standard_normal((2, 3, 64)).astype(np.float32)
    kc, vc = tn.zeros((3, 10, 64), "float32", "hip"), tn.zeros((3, 10, 64), "float32", "hip")
    pos = _dev(tn, np.array([8], np.int32))
    d_k, d_v = _dev(tn, k), _dev(tn, v)
    L.check(L.lib().tn_kv_append(None, d_k.data_ptr(), d_v.data_ptr(), 2, 3, 64, kc.data_ptr(), vc.data_ptr(), 10,
                                 pos.data_ptr()))
    gk, gv = kc.numpy(), vc.numpy()
    assert np.array_equal(gk[:, 8], k[0]) and np.array_equal(gk[:, 9], k[1])
    assert np.array_equal(gv[:, 8], v[0]) and np.array_equal(gv[:, 9], v[1])
    assert not gk[:, :8].any() and not gv[:, :8].any()


# max_len <= 1024 runs the single-pass kernel, above it the split-KV one
@pytest.mark.parametrize("D,hq,hkv,lens,cap", [(64, 9, 3, [1, 200, 300], 320), (128, 8, 2, [513, 17], 600),
                                              (64, 4, 2, [1500, 1, 1025], 1600), (128, 2, 1, [1024, 257], 1024)])
def test_f32_decode_attention_within_the_derived_bound(tn, D, hq, hkv, lens, cap):
    L = _lib()
    B = len(lens)
    rng = np.random.default_rng(D + cap)
    q = rng.standard_normal((B, hq, D)).astype(np.float32)
    kc = rng.standard_normal((B, hkv, cap, D)).astype(np.float32)
    vc = rng.standard_normal((B, hkv, cap, D)).astype(np.float32)
    out = tn.empty((B, hq, D), "float32", "hip")
    lse = tn.empty((B, hq), "float32", "hip")
    d_q, d_kc, d_vc, d_lens = _dev(tn, q), _dev(tn, kc), _dev(tn, vc), _dev(tn, np.asarray(lens, np.int32))
    L.check(L.lib().tn_sdpa_decode(None, L.TN_F32, d_q.data_ptr(), d_kc.data_ptr(), d_vc.data_ptr(), B, hq, hkv,
                                   cap, D, d_lens.data_ptr(), max(lens), float("nan"), out.data_ptr(),
                                   lse.data_ptr()))
    got, gl = out.numpy(), lse.numpy()
    for b in range(B):
        n = lens[b]
        args = (q[b:b + 1, :, None, :], kc[b:b + 1, :, :n], vc[b:b + 1, :, :n])
        r32, l32 = O.sdpa(*args)
        r64, l64 = O.sdpa(*[a.astype(np.float64) for a in args], dtype=np.float64)
        _within(got[b][None, :, None, :], r32.astype(np.float64), r64)
        _within(gl[b][None, :, None], l32.astype(np.float64), l64)


@pytest.mark.parametrize("k,n", [(576, 960), (1536, 576), (64, 3), (2304, 70)])
def test_fused_decode_linear_equals_the_separate_ops(tn, k, n):
    """tn_q4_0_linear_decode against tn_rmsnorm / tn_silu_mul, then
    tn_q4_0_linear, then tn_add: bit for bit, including y aliasing the
    residual. k = 2304 takes two batches of the activation loads."""
    from torchnative_amd import _C

    L = _lib()
    f = L.lib()
    rng = np.random.default_rng(k * 7 + n)
    w = _dev(tn, (rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    q = _C._quantize(w, "q4_0")
    qs, d = q._qs.data_ptr(), q._d.data_ptr()
    x = _dev(tn, (rng.standard_normal(2 * k) * 2).astype(np.float32))
    g = _dev(tn, rng.standard_normal(k).astype(np.float32))
    res = rng.standard_normal(n).astype(np.float32)
    d_res = _dev(tn, res)
    t = tn.empty((k,), "float32", "hip")
    ref, got = tn.empty((n,), "float32", "hip"), tn.empty((n,), "float32", "hip")

    def lin(src, out):
        L.check(f.tn_q4_0_linear(None, src, L.TN_F32, 1, k, qs, d, n, None, out.data_ptr(), L.TN_F32))

    L.check(f.tn_rmsnorm(None, x.data_ptr(), 1, k, g.data_ptr(), 1e-5, t.data_ptr()))
    lin(t.data_ptr(), ref)
    L.check(f.tn_q4_0_linear_decode(None, x.data_ptr(), k, L.TN_PRO_RMSNORM, g.data_ptr(), 1e-5, qs, d, n, None,
                                    got.data_ptr()))
    assert np.array_equal(got.numpy(), ref.numpy())

    L.check(f.tn_silu_mul(None, x.data_ptr(), x.data_ptr() + 4 * k, k, t.data_ptr()))
    lin(t.data_ptr(), ref)
    L.check(f.tn_q4_0_linear_decode(None, x.data_ptr(), k, L.TN_PRO_SILU, None, 0.0, qs, d, n, None,
                                    got.data_ptr()))
    assert np.array_equal(got.numpy(), ref.numpy())

    # residual epilogue, in place on the residual (the decoder's h += ...)
    lin(x.data_ptr(), ref)
    L.check(f.tn_add(None, d_res.data_ptr(), ref.data_ptr(), n, ref.data_ptr()))
    L.check(f.tn_q4_0_linear_decode(None, x.data_ptr(), k, L.TN_PRO_NONE, None, 0.0, qs, d, n, d_res.data_ptr(),
                                    d_res.data_ptr()))
    assert np.array_equal(d_res.numpy(), ref.numpy())
    # and the plain row equals tn_q4_0_linear
    lin(x.data_ptr(), ref)
    L.check(f.tn_q4_0_linear_decode(None, x.data_ptr(), k, L.TN_PRO_NONE, None, 0.0, qs, d, n, None,
                                    got.data_ptr()))
    assert np.array_equal(got.numpy(), ref.numpy())


@pytest.mark.parametrize("k,n", [(576, 1536), (1536, 576), (64, 3), (2304, 70), (128, 256)])
def test_fused_rmsnorm_silu_linear_equals_the_separate_ops(tn, k, n):
    """TN_PRO_RMSNORM_SILU (the decode step's gate_up launch) against
    tn_rmsnorm, tn_q4_0_linear over the stacked [gate; up] weight (2n rows)
    and tn_silu_mul of its two halves: bit for bit. A residual is refused."""
    from torchnative_amd import _C

    L = _lib()
    f = L.lib()
    rng = np.random.default_rng(k * 5 + n)
    w = _dev(tn, (rng.standard_normal((2 * n, k)) * 0.05).astype(np.float32))
    q = _C._quantize(w, "q4_0")
    qs, d = q._qs.data_ptr(), q._d.data_ptr()
    x = _dev(tn, (rng.standard_normal(k) * 2).astype(np.float32))
    g = _dev(tn, rng.standard_normal(k).astype(np.float32))
    t = tn.empty((k,), "float32", "hip")
    gu = tn.empty((2 * n,), "float32", "hip")
    ref, got = tn.empty((n,), "float32", "hip"), tn.empty((n,), "float32", "hip")
    L.check(f.tn_rmsnorm(None, x.data_ptr(), 1, k, g.data_ptr(), 1e-5, t.data_ptr()))
    L.check(f.tn_q4_0_linear(None, t.data_ptr(), L.TN_F32, 1, k, qs, d, 2 * n, None, gu.data_ptr(), L.TN_F32))
    L.check(f.tn_silu_mul(None, gu.data_ptr(), gu.data_ptr() + 4 * n, n, ref.data_ptr()))
    L.check(f.tn_q4_0_linear_decode(None, x.data_ptr(), k, L.TN_PRO_RMSNORM_SILU, g.data_ptr(), 1e-5, qs, d, n,
                                    None, got.data_ptr()))
    assert np.array_equal(got.numpy(), ref.numpy())
    assert f.tn_q4_0_linear_decode(None, x.data_ptr(), k, L.TN_PRO_RMSNORM_SILU, g.data_ptr(), 1e-5, qs, d, n,
                                   got.data_ptr(), got.data_ptr()) == L.TN_EINVAL


SMALL = OD.LlamaConfig(n_layers=2, hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, inter=256, vocab=512)
SMALL128 = OD.LlamaConfig(n_layers=2, hidden=256, n_heads=2, n_kv_heads=1, head_dim=128, inter=256, vocab=512)


# cap 24: the fused split attention merged in the o projection (head dim 64
# and 128); cap 600 (more than 16 splits of 32 keys): RoPE + append, split-KV
# attention and its combine
@pytest.mark.parametrize("cfg,cap", [(SMALL, 24), (SMALL, 600), (SMALL128, 24)], ids=["fused", "long", "fused-d128"])
def test_decode_step_matches_the_oracle_teacher_forced(tn, cfg, cap):
    """A 2-layer model: the GPU's logits at every step within the bound of the
    oracle's float32 run on the same tokens, and its greedy token the
    oracle's wherever the oracle's top two logits are further apart than
    the bound."""
    from torchnative_amd.decoder import Q4Llama

    prompt = [5, 77, 300, 12, 511, 0, 42, 9, 100, 250, 3, 64]
    n_new = 8
    model = Q4Llama(cfg, seed=11, cap=cap)
    ref32 = OD.Decoder(cfg, 11, cap, np.float32)
    ref64 = OD.Decoder(cfg, 11, cap, np.float64)
    model.start(prompt)
    seq = list(prompt)
    for pos in range(len(prompt) + n_new - 1):
        model.step()
        got = model.logits.numpy()
        token = seq[pos]
        l32 = ref32.step(token, pos).astype(np.float64)
        l64 = ref64.step(token, pos)
        tol = O.sdpa_tolerance(l32, l64, "float32")
        worst = float(np.max(np.abs(got - l32) / tol))
        assert worst <= 1.0, f"position {pos}: {worst:.3g}x the bound"
        nxt = int(model.state.numpy()[2])
        top = np.sort(l32)[-2:]
        if top[1] - top[0] > 2 * float(np.max(tol)):
            assert nxt == (seq[pos + 1] if pos + 1 < len(prompt) else OD.argmax(l32))
        if pos + 1 >= len(prompt):
            seq.append(nxt)
    assert model.generated(len(prompt), n_new) == seq[len(prompt):]


def test_graph_replay_equals_eager_steps(tn):
    """The captured steps are the same kernels on the same state: identical
    tokens and logits, bit for bit."""
    from torchnative_amd.decoder import Q4Llama
    from torchnative_amd import _lib as L

    prompt = [1, 2, 3, 4, 5, 6]
    model = Q4Llama(SMALL, seed=12, cap=20)
    eager = model.generate(prompt, 10)
    eager_logits = model.logits.numpy()
    s = ctypes.c_void_p()
    L.check(L.lib().tn_stream_create(ctypes.byref(s)))
    try:
        graphed = model.generate(prompt, 10, stream=s.value, graph=True)
        assert graphed == eager
        assert np.array_equal(model.logits.numpy(), eager_logits)
    finally:
        L.check(L.lib().tn_stream_destroy(s.value))
