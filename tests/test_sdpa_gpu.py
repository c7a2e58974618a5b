"""SDPA on the MI355X against the CPU oracle of the reference's default path.

Tolerance (written out in `_bound`): per output tensor, 4x the reference's own
fp32-vs-fp64 distance on the same inputs, floored at 1.186e-6 of the tensor's
scale (the reference's docs/numerics/AGREE.md section 2 rule). A bf16 run adds
one bf16 ulp of max(|ref|, |gpu|) (both sides round to bf16) and the
P-narrowing term u * sum_j P_ij |V_jd| with u = 2^-8, bf16's unit roundoff
(upstream's blocked kernel narrows P to bf16 between the products,
flash.rs:503-516). An f16 run adds one f16 ulp, the same term with u = 2^-11
and 2^-25 * sum_j |V_jd| over the attended keys (probabilities that round in
f16's subnormal range). The lse is compared in f32 with the same base rule.
"""

import math

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
OP = "aten._scaled_dot_product_flash_attention_for_cpu.default"


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


def _det(shape, seed):
    return np.array(O.sdpa_det(int(np.prod(shape)), seed), dtype=np.float64).reshape(shape)


def _bound(ref32, ref64, pav=None, bf16=False, got=None, kind=None, vsum=None):
    kind = kind or ("bfloat16" if bf16 else "float32")
    return O.sdpa_tolerance(ref32, ref64, kind, p=pav, got=got, vsum=vsum)


def _dev(tn, dtype, a):
    """A device tensor of `dtype` holding `a` rounded RNE to it."""
    if dtype == "float16":
        return tn.tensor(a.astype(np.float32).astype(np.float16), dtype="float16", device="hip")
    return tn.tensor(a.astype(np.float32), dtype=dtype, device="hip")


def _narrow(dtype, r32):
    """The oracle's f32 answer narrowed RNE to the output dtype, widened back."""
    if dtype == "bfloat16":
        return O.bf16_to_f32(O.bf16_from_f32(r32)).astype(np.float64)
    if dtype == "float16":
        return np.asarray(r32, np.float32).astype(np.float16).astype(np.float64)
    return np.asarray(r32, np.float64)


def _vsum(vw, Hq, L, causal, mask=None):
    """sum_j |V_jd| over the keys row i attends (upper-left causal, finite mask)."""
    B, Hkv, S, D = vw.shape
    av = np.repeat(np.abs(vw), Hq // Hkv, axis=1)
    att = np.ones((B, Hq, L, S))
    if causal:
        att = att * np.tril(np.ones((L, S)))
    if mask is not None:
        att = att * np.isfinite(mask)
    return att @ av


def _run(tn, dtype, q, k, v, causal, threads=16, scale=None):
    """GPU result plus the oracle's f32 and f64 answers on the same inputs."""
    B, Hq, L, D = q.shape
    qb, kb, vb = (_dev(tn, dtype, a) for a in (q, k, v))
    qw, kw, vw = (t.numpy().astype(np.float64) for t in (qb, kb, vb))  # exact widening
    o, lse = tn._aten_dispatch(OP, qb, kb, vb, 0.0, causal, scale=scale)
    r32, l32 = O.sdpa(qw, kw, vw, is_causal=causal, scale=scale, threads=threads)
    r64, l64 = O.sdpa(qw, kw, vw, is_causal=causal, scale=scale, threads=threads, dtype=np.float64)
    pav = vsum = None
    if dtype != "float32":
        pav, _ = O.sdpa(qw, kw, np.abs(vw), is_causal=causal, scale=scale, threads=threads, dtype=np.float64)
    if dtype == "float16":
        vsum = _vsum(vw, Hq, L, causal)
    return o, lse, (r32, l32, r64, l64, pav, vsum)


def _check(tn, dtype, q, k, v, causal, scale=None):
    o, lse, (r32, l32, r64, l64, pav, vsum) = _run(tn, dtype, q, k, v, causal, scale=scale)
    got = o.numpy().astype(np.float64)
    ref = _narrow(dtype, r32)
    tol = _bound(r32, r64, pav, got=got, kind=dtype, vsum=vsum) if dtype != "float32" else _bound(r32, r64)
    err = np.abs(got - ref)
    assert np.all(np.isfinite(got))
    worst = float(np.max(err / tol))
    assert worst <= 1.0, f"{dtype} causal={causal} {q.shape}x{k.shape}: {worst:.3g}x the bound, max err {err.max():.3g}"
    lt = _bound(l32, l64)
    lerr = float(np.max(np.abs(lse.numpy().astype(np.float64) - l32) / lt))
    assert lerr <= 1.0, f"lse {lerr:.3g}x the bound"
    return worst


SHAPES = [
    # (batch, q heads, kv heads, q_len, kv_len, head_dim)
    (1, 9, 3, 26, 26, 64),       # the reference's _SDPA_SHAPES entry with D=64 (test_shim.py:12077)
    (1, 2, 2, 33, 33, 64),       # second query block (cases.py:11430)
    (1, 2, 2, 70, 70, 128),      # three query blocks
    (1, 1, 1, 40, 600, 64),      # past the 512-key split (cases.py:11433)
    (2, 8, 2, 65, 130, 128),     # tails in both dims, batch 2, GQA 4
    (1, 4, 4, 2, 5, 64),         # q_len < kv_len: upper-left causal
    (1, 3, 1, 100, 37, 64),      # q_len > kv_len
]


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", SHAPES)
def test_sdpa_matches_the_oracle_within_the_derived_bound(tn, shape, causal, dtype):
    b, hq, hkv, l, s, d = shape
    q, k, v = _det((b, hq, l, d), 1), _det((b, hkv, s, d), 2), _det((b, hkv, s, d), 3)
    _check(tn, dtype, q, k, v, causal)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_config2_causal_gqa_prefill_at_full_size(tn, dtype):
    """B=1, 9 q heads / 3 kv heads, D=64, S=2048, causal,
    Q/K/V ~ N(0,1), scale 1/8."""
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 9, 2048, 64))
    k = rng.standard_normal((1, 3, 2048, 64))
    v = rng.standard_normal((1, 3, 2048, 64))
    worst = _check(tn, dtype, q, k, v, True)
    print(f"config 2 {dtype}: worst error {worst:.3f} of the bound", flush=True)


@pytest.mark.parametrize("shape,causal", [
    ((1, 1, 1, 64, 4096, 64), False),   # one query block of 64 key tiles: 64 workgroups, 64 partials
    ((1, 2, 1, 70, 3000, 128), False),  # two blocks per head of 94 32-key tiles, each cut into 94 partials
    ((1, 1, 1, 600, 600, 64), True),    # causal blocks of 1..10 tiles over 55 units, one per workgroup
])
def test_f32_stream_partition_cuts_blocks_into_many_partials(tn, shape, causal):
    """The f32 prefill cuts its (head, query block, key tile) units into
    equal ranges over the resident workgroups, at most one workgroup per
    unit. A short query range over long keys therefore splits each query
    block across dozens of workgroups; the combine merges them past its
    first batch of eight, in workgroup order."""
    b, hq, hkv, l, s, d = shape
    q, k, v = _det((b, hq, l, d), 11), _det((b, hkv, s, d), 12), _det((b, hkv, s, d), 13)
    _check(tn, "float32", q, k, v, causal)


def test_default_scale_and_explicit_scale_agree(tn):
    rng = np.random.default_rng(5)
    q, k, v = (tn.tensor(rng.standard_normal(s).astype(np.float32), device="hip")
               for s in ((1, 2, 16, 64), (1, 2, 16, 64), (1, 2, 16, 64)))
    a, la = tn._aten_dispatch(OP, q, k, v, 0.0, False)
    b, lb = tn._aten_dispatch(OP, q, k, v, 0.0, False, scale=1.0 / math.sqrt(64))
    assert np.array_equal(a.numpy(), b.numpy()) and np.array_equal(la.numpy(), lb.numpy())


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_negative_scale_runs_on_the_plain_kernel(tn, dtype):
    """The MFMA kernels take the row maximum of the unscaled scores, right
    only for scale >= 0; a negative scale runs on the plain kernel, whose
    maximum is over the scaled scores."""
    q, k, v = _det((1, 4, 70, 64), 41), _det((1, 2, 90, 64), 42), _det((1, 2, 90, 64), 43)
    _check(tn, dtype, q, k, v, True, scale=-0.125)
    _check(tn, dtype, q, k, v, False, scale=-0.3)


ANY_SHAPES = [
    # head dims the MFMA kernels do not take: the plain kernel
    (1, 4, 2, 40, 70, 32),
    (2, 3, 1, 33, 50, 80),
    (1, 6, 3, 17, 29, 72),
    (1, 2, 2, 100, 300, 96),
    (1, 2, 1, 20, 45, 256),
    (1, 2, 2, 7, 9, 1),
    (1, 3, 3, 70, 70, 200),
]


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", ANY_SHAPES)
def test_other_head_dims_match_the_oracle(tn, shape, causal, dtype):
    b, hq, hkv, l, s, d = shape
    q, k, v = _det((b, hq, l, d), 4), _det((b, hkv, s, d), 5), _det((b, hkv, s, d), 6)
    _check(tn, dtype, q, k, v, causal)


def test_head_dim_past_256_is_refused_by_name(tn):
    q = tn.tensor(np.ones((1, 1, 4, 264), np.float32), device="hip")
    with pytest.raises(NotImplementedError, match="head_dim 264"):
        tn._aten_dispatch(OP, q, q, q, 0.0, False)


def test_gqa_is_indexed_not_tiled(tn):
    """Query head i reads kv head i // n_rep: equal to running each head alone."""
    rng = np.random.default_rng(6)
    q = rng.standard_normal((1, 6, 20, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 20, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, 20, 64)).astype(np.float32)
    o, _ = tn._aten_dispatch(OP, *(tn.tensor(a, device="hip") for a in (q, k, v)), 0.0, True)
    full = o.numpy()
    for h in range(6):
        kh = h // 3
        oh, _ = tn._aten_dispatch(OP, tn.tensor(q[:, h:h + 1], device="hip"), tn.tensor(k[:, kh:kh + 1], device="hip"),
                                  tn.tensor(v[:, kh:kh + 1], device="hip"), 0.0, True)
        assert np.array_equal(oh.numpy()[:, 0], full[:, h])


def _decode_case(tn, B, Hq, Hkv, D, lens, cap, seed, max_len=None, scale=None, dtype="bfloat16"):
    """16-bit decode against the oracle per sequence; sequence b attends to
    keys 0 .. min(lens[b], max_len)-1 (a longer length is truncated at max_len)."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    kc = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    vc = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    qb, kb, vb = (_dev(tn, dtype, a) for a in (q, kc, vc))
    ln = tn.tensor(np.asarray(lens, np.int32), device="hip")
    max_len = max(lens) if max_len is None else max_len
    o, lse = tn.sdpa_decode(qb, kb, vb, ln, max_len, scale=scale)
    got = o.numpy().astype(np.float64)
    glse = lse.numpy().astype(np.float64)
    qw, kw, vw = (t.numpy().astype(np.float64) for t in (qb, kb, vb))
    worst = 0.0
    for b in range(B):
        L = min(lens[b], max_len)
        if L == 0:  # no keys: 0/0, as the split combine has always returned
            assert np.all(np.isnan(got[b])) and np.all(glse[b] == -np.inf)
            continue
        args = (qw[b:b + 1, :, None, :], kw[b:b + 1, :, :L], vw[b:b + 1, :, :L])
        r32, l32 = O.sdpa(*args, scale=scale)
        r64, l64 = O.sdpa(*args, scale=scale, dtype=np.float64)
        pav, _ = O.sdpa(args[0], args[1], np.abs(args[2]), scale=scale, dtype=np.float64)
        vsum = _vsum(args[2], Hq, 1, False) if dtype == "float16" else None
        ref = _narrow(dtype, r32)
        tol = _bound(r32, r64, pav, got=got[b:b + 1, :, None, :], kind=dtype, vsum=vsum)
        err = np.abs(got[b:b + 1, :, None, :] - ref)
        worst = max(worst, float(np.max(err / tol)))
        lt = _bound(l32, l64)
        assert float(np.max(np.abs(glse[b:b + 1, :, None] - l32) / lt)) <= 1.0
    assert worst <= 1.0, worst
    return worst


def test_decode_small_and_ragged(tn):
    _decode_case(tn, 3, 8, 2, 128, [1, 77, 300], 320, 7)
    _decode_case(tn, 2, 4, 4, 64, [129, 64], 200, 8)
    _decode_case(tn, 2, 16, 1, 128, [513, 5], 600, 9)


def test_decode_stream_partition_edges(tn):
    """The stream-K decode cuts all sequences' keys into equal ranges per wave:
    a range that starts or ends inside a sequence, one that covers many short
    sequences, empty sequences between them, a single key, and lengths past
    max_len (truncated)."""
    rng = np.random.default_rng(11)
    lens = [int(x) for x in rng.integers(0, 40, size=150)]
    lens[0], lens[1], lens[-1] = 0, 1, 0
    _decode_case(tn, 150, 8, 2, 128, lens, 48, 12)
    _decode_case(tn, 3, 4, 1, 64, [0, 1, 0], 8, 13)
    _decode_case(tn, 2, 4, 2, 64, [100, 50], 128, 14, max_len=64)


@pytest.mark.parametrize("hq,hkv,d", [(8, 1, 128), (9, 3, 64), (6, 6, 128), (16, 2, 64), (24, 4, 128)])
def test_decode_head_groups(tn, hq, hkv, d):
    """Query heads per kv head 8, 3, 1, 8 and 6 (groups of 8, 3, 1, 8 and 3 heads
    per wave)."""
    _decode_case(tn, 3, hq, hkv, d, [700, 33, 1500], 1536, 15 + hq)


def test_decode_f16_caches(tn):
    """float16 caches on both decode kernels: the stream-K one (ragged
    lengths, head groups of 8 and 3, a negative scale) and the per-split one
    (more than 1024 sequences), and BASELINE config 4's shape."""
    _decode_case(tn, 3, 8, 2, 128, [1, 77, 300], 320, 51, dtype="float16")
    _decode_case(tn, 2, 9, 3, 64, [129, 64], 200, 52, dtype="float16", scale=-0.2)
    rng = np.random.default_rng(53)
    lens = [int(x) for x in rng.integers(1, 20, size=1100)]
    _decode_case(tn, 1100, 2, 1, 64, lens, 24, 54, dtype="float16")
    lens = [int(x) for x in rng.integers(512, 4097, size=16)]
    _decode_case(tn, 16, 32, 8, 128, lens, 4096, 55, dtype="float16")


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_decode_other_head_dims(tn, dtype):
    """Head dims the MFMA decode kernels do not take run on the plain kernel,
    with ragged lengths, an empty sequence and truncation at max_len."""
    _decode_case(tn, 3, 8, 2, 96, [1, 77, 300], 320, 71, dtype=dtype)
    _decode_case(tn, 3, 4, 4, 32, [0, 5, 40], 48, 72, dtype=dtype)
    _decode_case(tn, 2, 6, 3, 80, [100, 50], 128, 73, max_len=64, dtype=dtype)
    _decode_case(tn, 2, 2, 1, 256, [33, 200], 200, 74, scale=-0.1, dtype=dtype)


def test_decode_scale_of_either_sign(tn):
    _decode_case(tn, 2, 8, 2, 128, [300, 41], 320, 21, scale=0.3)
    _decode_case(tn, 2, 8, 2, 128, [300, 41], 320, 22, scale=-0.2)


def test_decode_above_the_stream_partition_batch_limit(tn):
    """More than 1024 sequences take the per-split kernel."""
    rng = np.random.default_rng(23)
    lens = [int(x) for x in rng.integers(1, 20, size=1100)]
    _decode_case(tn, 1100, 2, 1, 64, lens, 24, 24)


def test_config4_decode_attention_at_full_size(tn):
    """B=16, 32 q heads / 8 kv heads, D=128, bf16, cache
    lengths uniform in [512, 4096]."""
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(512, 4097, size=16)]
    worst = _decode_case(tn, 16, 32, 8, 128, lens, 4096, 44)
    print(f"config 4: worst error {worst:.3f} of the bound", flush=True)


def _check_masked(tn, dtype, q, k, v, mask, mask_dtype, causal=False, nan_rows=()):
    """An additive mask (aten.rs:10383-10389) against the oracle, same bound
    as the unmasked runs. `mask` may be any shape broadcastable to
    [B, Hq, L, S]; rows listed in nan_rows are fully masked and must be NaN
    in out and lse, as the reference's are (aten.rs:10392-10420)."""
    B, Hq, L, D = q.shape
    S = k.shape[2]
    qt, kt, vt = (_dev(tn, dtype, a) for a in (q, k, v))
    mt = _dev(tn, mask_dtype, mask)
    o, lse = tn._aten_dispatch(OP, qt, kt, vt, 0.0, causal, attn_mask=mt)
    qw, kw, vw = (t.numpy().astype(np.float64) for t in (qt, kt, vt))
    mw = np.ascontiguousarray(np.broadcast_to(mt.numpy().astype(np.float64), (B, Hq, L, S)))
    with np.errstate(invalid="ignore"):
        r32, l32 = O.sdpa(qw, kw, vw, mask=mw, is_causal=causal, threads=16)
        r64, l64 = O.sdpa(qw, kw, vw, mask=mw, is_causal=causal, threads=16, dtype=np.float64)
        pav = O.sdpa(qw, kw, np.abs(vw), mask=mw, is_causal=causal, threads=16, dtype=np.float64)[0] \
            if dtype != "float32" else None
    vsum = _vsum(vw, Hq, L, causal, mw) if dtype == "float16" else None
    got, gl = o.numpy().astype(np.float64), lse.numpy().astype(np.float64)
    nan = np.zeros((B, Hq, L), bool)
    for (b, h, i) in nan_rows:
        nan[b, h, i] = True
    assert np.array_equal(np.isnan(got).any(axis=-1), nan) and np.all(np.isnan(got[nan]))
    assert np.array_equal(np.isnan(gl), nan)
    keep = ~nan
    ref = _narrow(dtype, r32)
    if dtype != "float32":
        tol = _bound(r32[keep], r64[keep], pav[keep], got=got[keep], kind=dtype,
                     vsum=vsum[keep] if vsum is not None else None)
    else:
        tol = _bound(r32[keep], r64[keep])
    worst = float(np.max(np.abs(got[keep] - ref[keep]) / tol))
    assert worst <= 1.0, f"{dtype} mask {mask_dtype} causal={causal}: {worst:.3g}x the bound"
    lt = _bound(l32[keep], l64[keep])
    assert float(np.max(np.abs(gl[keep] - l32[keep]) / lt)) <= 1.0


@pytest.mark.parametrize("dtype,mask_dtype,D,causal", [
    ("bfloat16", "float32", 64, False), ("bfloat16", "bfloat16", 64, True), ("bfloat16", "float32", 128, True),
    ("float32", "float32", 64, True), ("float32", "float32", 128, False),
    ("float16", "float16", 64, True), ("float16", "float32", 128, False),
    ("float16", "float16", 80, False), ("bfloat16", "float32", 96, True), ("float32", "float32", 32, False)])
def test_additive_mask_within_the_derived_bound(tn, dtype, mask_dtype, D, causal):
    rng = np.random.default_rng(D + int(causal))
    B, Hq, Hkv, L, S = 2, 4, 2, 70, 90
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, L, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    mask = rng.standard_normal((B, Hq, L, S)) * 2
    mask[rng.random(mask.shape) < 0.1] = -np.inf  # a sprinkle of masked keys (never a whole row here)
    mask[:, :, :, 0] = 0.0
    _check_masked(tn, dtype, q, k, v, mask, mask_dtype, causal)


def test_broadcast_mask_and_fully_masked_rows(tn):
    rng = np.random.default_rng(7)
    B, Hq, Hkv, L, S, D = 1, 3, 1, 40, 65, 64
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, L, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    mask = np.where(rng.random((L, S)) < 0.3, -np.inf, 0.0)  # [L, S], broadcast over batch and heads
    mask[:, 5] = 0.0
    mask[17, :] = -np.inf  # row 17 of every head sees no key
    _check_masked(tn, "bfloat16", q, k, v, mask, "float32", nan_rows=[(0, h, 17) for h in range(Hq)])


def test_mask_on_split_rows_merged_in_kernel(tn):
    """Rows of 2048 keys are split across workgroups and merged inside the
    kernel; the mask is applied in every split."""
    rng = np.random.default_rng(9)
    B, Hq, Hkv, L, S, D = 1, 2, 1, 128, 2048, 64
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, L, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    mask = rng.standard_normal((B, Hq, L, S))
    mask[:, :, :, 1024:1500] = -np.inf
    _check_masked(tn, "bfloat16", q, k, v, mask, "bfloat16")


def test_f16_split_rows_with_an_f16_mask_and_a_fully_masked_row(tn):
    """float16 through the in-kernel merge of split rows, with a float16 mask
    that leaves one row with no key (NaN) and takes most of another."""
    rng = np.random.default_rng(31)
    B, Hq, Hkv, L, S, D = 1, 4, 2, 96, 2048, 128
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, L, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    mask = rng.standard_normal((B, Hq, L, S))
    mask[:, :, 40, :] = -np.inf
    mask[:, :, 41, 3:] = -np.inf
    _check_masked(tn, "float16", q, k, v, mask, "float16", nan_rows=[(0, h, 40) for h in range(Hq)])


def test_f16_large_values_narrow_without_overflow(tn):
    """Inputs near f16's range: scores are formed in f32 (no overflow), the
    output lands in range and is narrowed RNE."""
    rng = np.random.default_rng(32)
    q = rng.standard_normal((1, 2, 64, 64)) * 200.0
    k = rng.standard_normal((1, 2, 64, 64)) * 200.0
    v = rng.standard_normal((1, 2, 64, 64)) * 3000.0
    _check(tn, "float16", q, k, v, True)


def test_mask_dtype_rule(tn):
    qt = tn.tensor(np.zeros((1, 1, 4, 64), np.float32), device="hip")
    mt = tn.tensor(np.zeros((1, 1, 4, 4), np.float32), dtype="bfloat16", device="hip")
    with pytest.raises(RuntimeError, match="Attention mask is the same data type as query"):
        tn._aten_dispatch(OP, qt, qt, qt, 0.0, False, attn_mask=mt)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_large_scores_on_the_mfma_kernels(tn, dtype, D, causal):
    """Scores far outside the usual range (q and k scaled by 20 and 200): the
    row maximum must be taken over finished MFMA results, or a partly
    accumulated maximum makes exp2 overflow. Every tile count from one to many
    stages and split rows (S up to 1100)."""
    for S, amp in ((64, 200.0), (100, 200.0), (300, 20.0), (1100, 20.0)):
        rng = np.random.default_rng(S + D)
        q = rng.standard_normal((1, 2, S, D)) * amp
        k = rng.standard_normal((1, 2, S, D)) * amp
        v = rng.standard_normal((1, 2, S, D)) * 30.0
        _check(tn, dtype, q, k, v, causal)


def test_large_scores_on_the_f32_and_decode_kernels(tn):
    rng = np.random.default_rng(61)
    for D in (64, 128):
        q = rng.standard_normal((1, 2, 300, D)) * 20.0
        k = rng.standard_normal((1, 2, 300, D)) * 20.0
        v = rng.standard_normal((1, 2, 300, D))
        _check(tn, "float32", q, k, v, True)
    # decode over bf16 and f16 caches: q and k scaled by 20 through the scale
    for dtype in ("bfloat16", "float16"):
        _decode_case(tn, 3, 8, 2, 128, [1, 77, 300], 320, 62, scale=400.0 / np.sqrt(128), dtype=dtype)
        _decode_case(tn, 2, 9, 3, 64, [700, 64], 800, 63, scale=400.0 / 8, dtype=dtype)


def _f64_bound(q, k, v, scale=None):
    """|gpu - oracle| for two f64 evaluations of the same attention: each is
    within 2 gamma_D * max_j sum_d |q_d k_jd| * |scale| * max|V| (score
    rounding, which moves each probability by at most that relative amount)
    plus 4 gamma_(S+4) * max|V| (the sums) of the exact value; the bound is
    twice that. The lse gets the score term without max|V| plus 4 gamma_(S+4)."""
    B, Hq, L, D = q.shape
    S = k.shape[2]
    g = lambda n: n * 2.0 ** -53 / (1 - n * 2.0 ** -53)
    kk = np.repeat(np.abs(k), Hq // k.shape[1], axis=1)
    amax = float(np.max(np.abs(q) @ np.swapaxes(kk, -1, -2)))
    sc = abs(scale) if scale is not None else 1.0 / np.sqrt(D)
    vmax = float(np.max(np.abs(v)))
    score = 2 * g(D) * amax * sc
    return 2 * (score * vmax + 4 * g(S + 4) * vmax), 2 * (score + 4 * g(S + 4))


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 9, 3, 26, 26, 64), (2, 8, 2, 65, 130, 128), (1, 3, 1, 100, 37, 80),
                                   (1, 2, 2, 40, 600, 64)])
def test_float64_computes_in_float64(tn, shape, causal):
    """f64 attention runs in f64: within the f64 rounding bound of the
    oracle's f64 result (an f32 evaluation misses it by orders of magnitude)."""
    b, hq, hkv, l, s, d = shape
    q, k, v = _det((b, hq, l, d), 7), _det((b, hkv, s, d), 8), _det((b, hkv, s, d), 9)
    qt, kt, vt = (tn.tensor(a, dtype="float64", device="hip") for a in (q, k, v))
    o, lse = tn._aten_dispatch(OP, qt, kt, vt, 0.0, causal)
    r64, l64 = O.sdpa(q, k, v, is_causal=causal, threads=16, dtype=np.float64)
    r32, _ = O.sdpa(q, k, v, is_causal=causal, threads=16)
    tol, ltol = _f64_bound(q, k, v)
    got = o.numpy()
    assert o.dtype == "float64" and lse.dtype == "float64"
    assert float(np.max(np.abs(got - r64))) <= tol
    assert float(np.max(np.abs(lse.numpy() - l64))) <= ltol
    assert float(np.max(np.abs(r32 - r64))) > tol  # the bound separates f64 from f32 arithmetic


def test_float64_mask_rule_and_masked_rows(tn):
    rng = np.random.default_rng(81)
    q, k, v = rng.standard_normal((1, 2, 20, 64)), rng.standard_normal((1, 2, 30, 64)), rng.standard_normal((1, 2, 30, 64))
    mask = rng.standard_normal((1, 2, 20, 30))
    mask[0, :, 4, :] = -np.inf
    qt, kt, vt = (tn.tensor(a, dtype="float64", device="hip") for a in (q, k, v))
    m32 = tn.tensor(mask.astype(np.float32), device="hip")
    with pytest.raises(NotImplementedError, match="float32 attn_mask on a float64"):
        tn._aten_dispatch(OP, qt, kt, vt, 0.0, False, attn_mask=m32)
    m64 = tn.tensor(mask, dtype="float64", device="hip")
    o, lse = tn._aten_dispatch(OP, qt, kt, vt, 0.0, False, attn_mask=m64)
    with np.errstate(invalid="ignore"):
        r64, l64 = O.sdpa(q, k, v, mask=mask, threads=16, dtype=np.float64)
    got = o.numpy()
    assert np.all(np.isnan(got[0, :, 4])) and np.all(np.isnan(lse.numpy()[0, :, 4]))
    keep = np.ones(20, bool)
    keep[4] = False
    tol, _ = _f64_bound(q, k, v)
    assert float(np.max(np.abs(got[0, :, keep] - r64[0, :, keep]))) <= tol + 2 ** -40 * float(np.max(np.abs(mask[np.isfinite(mask)])))
