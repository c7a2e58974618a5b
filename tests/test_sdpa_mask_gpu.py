"""Attention masks on the MI355X: bool masks and masks broadcast by strides.

F.scaled_dot_product_attention turns a bool mask into the additive
where(mask, 0, -inf) in the query's dtype before the flash op
(bootstrap.py:12918-12925, :13065-13066); the flash op broadcasts a smaller
mask onto [B, Hq, L, S] (aten.rs:10293-10303). Here the kernels read both in
place: the bool bytes and the mask's own storage through zero strides. The
oracle gets the additive mask, broadcast to the full shape, so it checks the
conversion and the broadcast together.

Tolerance: the rule of tests/test_sdpa_gpu.py (`_check_masked`), i.e. 4x the
reference's own fp32-vs-fp64 distance floored at 1.186e-6 of the tensor's
scale, plus one output ulp and the P-narrowing term for 16-bit dtypes.
"""

import numpy as np
import pytest

import oracle as O

from test_sdpa_gpu import OP, _bound, _dev, _f64_bound, _narrow, _vsum

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


def _bool_case(tn, dtype, q, k, v, mask, nan_rows=()):
    """F.sdpa with the bool `mask` (any shape broadcastable to [B, Hq, L, S])
    against the oracle's run with where(mask, 0, -inf)."""
    B, Hq, L, D = q.shape
    S = k.shape[2]
    qt, kt, vt = (_dev(tn, dtype, a) for a in (q, k, v))
    mt = tn.tensor(np.asarray(mask, bool), device="hip")
    enable_gqa = Hq != k.shape[1]
    o = tn.scaled_dot_product_attention(qt, kt, vt, attn_mask=mt, enable_gqa=enable_gqa)
    qw, kw, vw = (t.numpy().astype(np.float64) for t in (qt, kt, vt))
    add = np.where(np.broadcast_to(np.asarray(mask, bool), (B, Hq, L, S)), 0.0, -np.inf)
    add = np.ascontiguousarray(add)
    with np.errstate(invalid="ignore"):
        r32, _ = O.sdpa(qw, kw, vw, mask=add, threads=16)
        r64, _ = O.sdpa(qw, kw, vw, mask=add, threads=16, dtype=np.float64)
        pav = O.sdpa(qw, kw, np.abs(vw), mask=add, threads=16, dtype=np.float64)[0] \
            if dtype in ("bfloat16", "float16") else None
    vsum = _vsum(vw, Hq, L, False, add) if dtype == "float16" else None
    got = o.numpy().astype(np.float64)
    nan = np.zeros((B, Hq, L), bool)
    for (b, h, i) in nan_rows:
        nan[b, h, i] = True
    assert np.array_equal(np.isnan(got).any(axis=-1), nan)
    keep = ~nan
    ref = _narrow(dtype, r32) if dtype != "float64" else r64
    if dtype in ("bfloat16", "float16"):
        tol = _bound(r32[keep], r64[keep], pav[keep], got=got[keep], kind=dtype,
                     vsum=vsum[keep] if vsum is not None else None)
    elif dtype == "float64":
        # two f64 evaluations: the derived f64 rounding bound of test_sdpa_gpu
        tol = _f64_bound(qw, kw, vw)[0]
    else:
        tol = _bound(r32[keep], r64[keep])
    worst = float(np.max(np.abs(got[keep] - ref[keep]) / tol))
    assert worst <= 1.0, f"{dtype} bool mask {np.shape(mask)}: {worst:.3g}x the bound"
    return worst


@pytest.mark.parametrize("dtype,D", [("bfloat16", 64), ("bfloat16", 128), ("float16", 64), ("float16", 128),
                                     ("float32", 64), ("float32", 128), ("bfloat16", 80), ("float64", 64)])
@pytest.mark.parametrize("shape", ["full", "LS", "B1LS", "B11S"])
def test_bool_mask_broadcast_in_place(tn, dtype, D, shape):
    rng = np.random.default_rng(D * 7 + len(shape))
    B, Hq, Hkv, L, S = 2, 6, 2, 72, 136
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, L, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    mshape = {"full": (B, Hq, L, S), "LS": (L, S), "B1LS": (B, 1, L, S), "B11S": (B, 1, 1, S)}[shape]
    mask = rng.random(mshape) < 0.7
    mask[..., 3] = True  # every row keeps a key
    _bool_case(tn, dtype, q, k, v, mask)


def test_bool_key_padding_mask_like_a_batch_of_prompts(tn):
    """The usual bool mask of batched generation: [B, 1, 1, S] with each
    sequence's padding masked, at a split-row length (S = 2048, bf16)."""
    rng = np.random.default_rng(5)
    B, Hq, Hkv, L, S, D = 2, 9, 3, 64, 2048, 64
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, L, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    mask = np.ones((B, 1, 1, S), bool)
    mask[0, ..., 1500:] = False
    mask[1, ..., :37] = False
    _bool_case(tn, "bfloat16", q, k, v, mask)


def test_bool_mask_with_a_row_that_sees_nothing(tn):
    rng = np.random.default_rng(6)
    B, Hq, Hkv, L, S, D = 1, 2, 1, 40, 64, 128
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, L, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    mask = rng.random((L, S)) < 0.5
    mask[:, 9] = True
    mask[11, :] = False
    _bool_case(tn, "float16", q, k, v, mask, nan_rows=[(0, h, 11) for h in range(Hq)])


def test_odd_key_length_reads_every_element_of_an_unaligned_row(tn):
    """S = 67: mask rows start at every alignment, so the vector reads fall
    back to element reads on most rows and on the last partial quad."""
    rng = np.random.default_rng(8)
    B, Hq, Hkv, L, S, D = 1, 3, 3, 50, 67, 64
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, L, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    mask = rng.random((B, Hq, L, S)) < 0.6
    mask[..., 66] = True
    _bool_case(tn, "bfloat16", q, k, v, mask)


@pytest.mark.parametrize("mshape", [(1, 1, 72, 136), (2, 1, 72, 136), (1, 6, 1, 136), (72, 1)])
def test_additive_mask_broadcast_by_strides(tn, mshape):
    """An f32 additive mask of a broadcastable shape is read where it lies
    (no host copy): against the oracle with the mask broadcast in numpy."""
    from test_sdpa_gpu import _check_masked

    rng = np.random.default_rng(sum(mshape))
    B, Hq, Hkv, L, S, D = 2, 6, 2, 72, 136, 64
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, L, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    mask = rng.standard_normal(mshape) * 2
    _check_masked(tn, "bfloat16", q, k, v, mask, "float32")


def test_the_flash_op_itself_refuses_a_bool_mask(tn):
    """The conversion belongs to F.sdpa: the aten op keeps the reference's
    dtype rule (aten.rs:10142-10148)."""
    qt = tn.tensor(np.zeros((1, 1, 4, 64), np.float32), device="hip")
    mt = tn.tensor(np.ones((1, 1, 4, 4), bool), device="hip")
    with pytest.raises(RuntimeError, match="Attention mask is the same data type as query"):
        tn._aten_dispatch(OP, qt, qt, qt, 0.0, False, attn_mask=mt)


def test_a_mask_that_does_not_broadcast_is_refused(tn):
    qt = tn.tensor(np.zeros((1, 2, 4, 64), np.float32), device="hip")
    mt = tn.tensor(np.zeros((3, 4), np.float32), device="hip")
    with pytest.raises(RuntimeError, match="cannot be broadcast"):
        tn._aten_dispatch(OP, qt, qt, qt, 0.0, False, attn_mask=mt)


# A mask that is the same for every query row ([B, 1, 1, S] key padding, or a
# per-head key bias [B, Hq, 1, S]) runs at head dim 64 on the kernel without
# split rows, which stages the 256 mask values of each ring stage in LDS;
# the shapes below give partial stages and tiles (S = 333), GQA, and causal
# rows on top of the mask.
@pytest.mark.parametrize("dtype,mask_dtype,mshape,causal", [
    ("bfloat16", "float32", (2, 1, 1, 333), True),
    ("bfloat16", "bfloat16", (1, 4, 1, 333), False),
    ("float16", "float16", (2, 4, 1, 333), True),
    ("float16", "float32", (1, 1, 1, 333), False),
])
def test_key_mask_on_the_kernel_without_split_rows(tn, dtype, mask_dtype, mshape, causal):
    from test_sdpa_gpu import _check_masked

    rng = np.random.default_rng(sum(mshape) + causal)
    B, Hq, Hkv, L, S, D = 2, 4, 2, 200, 333, 64
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, L, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    mask = rng.standard_normal(mshape) * 2
    mask[..., 50:60] = -np.inf  # keys no row may see
    _check_masked(tn, dtype, q, k, v, mask, mask_dtype, causal)


def test_key_padding_in_front_leaves_the_first_causal_rows_empty(tn):
    """Keys 0-36 masked and causal rows: rows 0-36 see no key, so their
    outputs and lse are NaN, as the reference's are."""
    from test_sdpa_gpu import _check_masked

    rng = np.random.default_rng(21)
    B, Hq, Hkv, L, S, D = 1, 3, 1, 100, 100, 64
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, L, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    mask = np.zeros((1, 1, 1, S))
    mask[..., :37] = -np.inf
    _check_masked(tn, "bfloat16", q, k, v, mask, "float32", causal=True,
                  nan_rows=[(0, h, i) for h in range(Hq) for i in range(37)])


def test_bool_key_padding_with_causal_rows_through_the_c_abi(tn):
    """The bench's masked leg: config 2's shape (bf16, causal, 9/3 heads,
    S = 2048) with a bool [B, 1, 1, S] mask hiding the last 64 keys, passed
    by strides to tn_sdpa_fwd, against the oracle with where(mask, 0, -inf)."""
    import ctypes

    from torchnative_amd import _lib as L
    from test_sdpa_gpu import _bound, _dev, _narrow

    rng = np.random.default_rng(22)
    B, Hq, Hkv, S, D = 1, 9, 3, 2048, 64
    q, k, v = (rng.standard_normal(s) for s in ((B, Hq, S, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    keep = np.ones((B, 1, 1, S), bool)
    keep[..., S - 64:] = False
    qt, kt, vt = (_dev(tn, "bfloat16", a) for a in (q, k, v))
    mt = tn.tensor(keep, device="hip")
    out = tn.empty((B, Hq, S, D), "bfloat16", "hip")
    lse = tn.empty((B, Hq, S), "float32", "hip")
    strides = (ctypes.c_int64 * 4)(S, 0, 0, 1)
    L.check(L.lib().tn_sdpa_fwd(None, L.TN_BF16, qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), B, Hq, Hkv, S, S, D,
                                mt.data_ptr(), L.TN_BOOL, strides, 1, float("nan"), out.data_ptr(),
                                lse.data_ptr()))
    qw, kw, vw = (t.numpy().astype(np.float64) for t in (qt, kt, vt))
    add = np.ascontiguousarray(np.broadcast_to(np.where(keep, 0.0, -np.inf), (B, Hq, S, S)))
    r32, l32 = O.sdpa(qw, kw, vw, mask=add, is_causal=True, threads=16)
    r64, l64 = O.sdpa(qw, kw, vw, mask=add, is_causal=True, threads=16, dtype=np.float64)
    pav = O.sdpa(qw, kw, np.abs(vw), mask=add, is_causal=True, threads=16, dtype=np.float64)[0]
    got, gl = out.numpy().astype(np.float64), lse.numpy().astype(np.float64)
    tol = _bound(r32, r64, pav, got=got, kind="bfloat16")
    assert float(np.max(np.abs(got - _narrow("bfloat16", r32)) / tol)) <= 1.0
    assert float(np.max(np.abs(gl - l32) / _bound(l32, l64))) <= 1.0
