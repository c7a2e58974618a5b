"""tn_sdpa_decode_noalloc: the decode attention with its work buffer in a
fixed device array, for callers that cannot allocate.

Checked against tn_sdpa_decode, which shares its kernels, bit for bit, on
two calls in a row (the second smaller, so stale contents of the array from
the first must not leak into it), on the stream-K path (bf16 and f16 caches),
the split path of f32 caches, and a path that needs no buffer; the library's
workspace counter shows the no-alloc calls allocate nothing; a call whose
buffer would not fit the array is refused by name.
"""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


def _case(tn, dtype, B, Hq, Hkv, D, cap, lens, seed):
    rng = np.random.default_rng(seed)
    mk = lambda shape: tn.tensor(rng.standard_normal(shape).astype(np.float32), dtype=dtype, device="hip")
    return dict(q=mk((B, Hq, D)), k=mk((B, Hkv, cap, D)), v=mk((B, Hkv, cap, D)),
                lens=tn.tensor(np.asarray(lens, np.int32), device="hip"), B=B, Hq=Hq, Hkv=Hkv, D=D, cap=cap,
                max_len=int(max(lens)), dtype=dtype)


def _run(tn, fn, c, stream):
    from torchnative_amd import _lib as L

    out = tn.empty((c["B"], c["Hq"], c["D"]), c["dtype"], "hip")
    lse = tn.empty((c["B"], c["Hq"]), "float32", "hip")
    code = {"bfloat16": L.TN_BF16, "float16": L.TN_F16, "float32": L.TN_F32}[c["dtype"]]
    L.check(fn(stream, code, c["q"].data_ptr(), c["k"].data_ptr(), c["v"].data_ptr(), c["B"], c["Hq"], c["Hkv"],
               c["cap"], c["D"], c["lens"].data_ptr(), c["max_len"], float("nan"), out.data_ptr(), lse.data_ptr()))
    L.check(L.lib().tn_stream_synchronize(stream))
    return out.bits(), lse.numpy()


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_noalloc_equals_the_allocating_entry_on_two_calls_in_a_row(tn, dtype):
    from torchnative_amd import _lib as L

    f = L.lib()
    rng = np.random.default_rng(1)
    if dtype == "float32":  # f32 caches longer than 1024 keys take the split kernel and its partials
        big = _case(tn, dtype, 4, 16, 4, 128, 2100, [2100, 1500, 7, 1025], 11)
        small = _case(tn, dtype, 2, 8, 2, 64, 1300, [1300, 1100], 12)
    else:  # config 4's shape, then a smaller one
        big = _case(tn, dtype, 16, 32, 8, 128, 4096, [int(x) for x in rng.integers(512, 4097, 16)], 13)
        small = _case(tn, dtype, 3, 9, 3, 64, 300, [300, 65, 1], 14)
    s = ctypes.c_void_p()
    L.check(f.tn_stream_create(ctypes.byref(s)))
    try:
        for c in (big, small):
            before = tn._hip_counters()["workspace_bytes"]
            got = _run(tn, f.tn_sdpa_decode_noalloc, c, s.value)
            assert tn._hip_counters()["workspace_bytes"] == before  # no work buffer was allocated
            want = _run(tn, f.tn_sdpa_decode, c, s.value)
            assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1]), (dtype, c["B"])
    finally:
        L.check(f.tn_stream_destroy(s.value))


def test_noalloc_on_a_path_without_a_work_buffer(tn):
    """Head dim 80 runs the plain kernel, which needs no buffer."""
    from torchnative_amd import _lib as L

    c = _case(tn, "bfloat16", 2, 4, 2, 80, 100, [100, 33], 15)
    got = _run(tn, L.lib().tn_sdpa_decode_noalloc, c, None)
    want = _run(tn, L.lib().tn_sdpa_decode, c, None)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


def test_noalloc_refuses_a_call_larger_than_its_array(tn):
    """1024 sequences of 16 heads: the stream-K partials need more than the
    array's 8 MiB (the buffers are real and sized, so even a call that ran
    would stay in bounds)."""
    from torchnative_amd import _lib as L

    c = _case(tn, "bfloat16", 1024, 16, 16, 128, 16, [16] * 1024, 16)
    with pytest.raises(ValueError, match="more than the 8388608 bytes of the fixed device array"):
        _run(tn, L.lib().tn_sdpa_decode_noalloc, c, None)
