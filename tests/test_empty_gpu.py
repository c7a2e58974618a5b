"""Empty inputs through the Python mirror on the MI355X: a quantised linear
with no activation rows gives a [0, N] output in each weight format, and the
SDPA op with no query rows gives empty outputs (aten.rs:10242-10259). Neither
launches a kernel or touches a null device pointer.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

OP = "aten._scaled_dot_product_flash_attention_for_cpu.default"


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


@pytest.mark.parametrize("fmt,k", [("q4_0", 64), ("q8_0", 64), ("q4_k", 256)])
@pytest.mark.parametrize("x_dtype", ["float32", "bfloat16"])
def test_linear_with_no_rows_gives_an_empty_output(tn, fmt, k, x_dtype):
    n = 24
    w = np.random.default_rng(5).standard_normal((n, k)).astype(np.float32)
    q = tn._quantize(tn.tensor(w, device="hip"), fmt)
    x = tn.tensor(np.zeros((0, k), np.float32), dtype=x_dtype, device="hip")
    y = tn._quantized_linear(x, q)
    assert tuple(y.shape) == (0, n)
    assert y.numpy().shape == (0, n)
    # a real row still goes through afterwards
    x1 = tn.tensor(np.ones((1, k), np.float32), dtype=x_dtype, device="hip")
    assert np.isfinite(tn._quantized_linear(x1, q).numpy()).all()


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_sdpa_with_no_query_rows_gives_empty_outputs(tn, dtype):
    B, Hq, Hkv, S, D = 1, 4, 2, 16, 64
    rng = np.random.default_rng(9)
    q = tn.tensor(np.zeros((B, Hq, 0, D), np.float32), dtype=dtype, device="hip")
    k = tn.tensor(rng.standard_normal((B, Hkv, S, D)).astype(np.float32), dtype=dtype, device="hip")
    v = tn.tensor(rng.standard_normal((B, Hkv, S, D)).astype(np.float32), dtype=dtype, device="hip")
    o, lse = tn._aten_dispatch(OP, q, k, v, 0.0, False)
    assert tuple(o.shape) == (B, Hq, 0, D)
    assert o.numpy().size == 0
    assert lse.numpy().size == 0
