"""Device residency and graph capture on the MI355X.

Residency is proven by the counters, as the reference proves its mps path
(tests/devices/mps/test_paged_attention.py:1-14, `host_downloads == 0`
across the dispatch): a masked SDPA (bool and broadcast additive masks), a
q4 linear (the GEMV and the GEMM) and decode steps of the fused Llama step
make no host readback at all.

Capture: any entry point can be recorded on a created stream
(tn_stream_begin_capture / tn_stream_end_capture) once a call of its shape
has run; a first call, which would allocate the stream's work buffers, is
refused by name while capturing. Replays are checked against the eager
result every time, with eager work in between.
"""

import ctypes

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


def test_no_host_readback_across_masked_sdpa_q4_linear_and_decode_steps(tn):
    from oracle import decoder as OD
    from torchnative_amd.decoder import Q4Llama

    rng = np.random.default_rng(3)
    q = tn.tensor(rng.standard_normal((2, 6, 96, 64)).astype(np.float32), dtype="bfloat16", device="hip")
    k = tn.tensor(rng.standard_normal((2, 2, 160, 64)).astype(np.float32), dtype="bfloat16", device="hip")
    v = tn.tensor(rng.standard_normal((2, 2, 160, 64)).astype(np.float32), dtype="bfloat16", device="hip")
    bmask = tn.tensor(rng.random((2, 1, 1, 160)) < 0.8, device="hip")
    amask = tn.tensor(rng.standard_normal((96, 160)).astype(np.float32), device="hip")
    x1 = tn.tensor(rng.standard_normal((1, 576)).astype(np.float32), device="hip")
    x2 = tn.tensor(rng.standard_normal((64, 576)).astype(np.float32), dtype="bfloat16", device="hip")
    w = tn._quantized_from_blob(O.synth_q4_0_weight(512, 576, 0.02, 4), (512, 576), "q4_0", device="hip")
    cfg = OD.LlamaConfig(n_layers=2, hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, inter=256, vocab=512)
    model = Q4Llama(cfg, seed=3, cap=40)
    model.start([1, 2, 3, 4])
    tn.synchronize()

    tn._C._hip_counters_reset()
    outs = [
        tn.scaled_dot_product_attention(q, k, v, attn_mask=bmask, enable_gqa=True),
        tn._aten_dispatch("aten._scaled_dot_product_flash_attention_for_cpu.default", q, k, v, 0.0, False,
                          attn_mask=amask)[0],
        tn._quantized_linear(x1, w),
        tn._quantized_linear(x2, w),
    ]
    for _ in range(6):
        model.step()
    tn.synchronize()
    c = tn._hip_counters()
    assert c["host_downloads"] == 0 and c["bytes_downloaded"] == 0, c
    assert c["dispatches"] >= 4 + 6, c
    assert len(outs) == 4


def _stream(tn):
    from torchnative_amd import _lib as L

    s = ctypes.c_void_p()
    L.check(L.lib().tn_stream_create(ctypes.byref(s)))
    return s.value


def test_capture_refuses_a_call_that_would_allocate_then_replays_what_it_recorded(tn):
    from torchnative_amd import _lib as L

    f = L.lib()
    rng = np.random.default_rng(9)
    B, Hq, Hkv, cap, D = 4, 8, 2, 700, 128
    q = tn.tensor(rng.standard_normal((B, Hq, D)).astype(np.float32), dtype="bfloat16", device="hip")
    kc = tn.tensor(rng.standard_normal((B, Hkv, cap, D)).astype(np.float32), dtype="bfloat16", device="hip")
    vc = tn.tensor(rng.standard_normal((B, Hkv, cap, D)).astype(np.float32), dtype="bfloat16", device="hip")
    lens = tn.tensor(np.array([700, 3, 250, 64], np.int32), device="hip")
    out = tn.empty((B, Hq, D), "bfloat16", "hip")
    lse = tn.empty((B, Hq), "float32", "hip")
    st = _stream(tn)
    try:
        def call():
            return f.tn_sdpa_decode(st, L.TN_BF16, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), B, Hq, Hkv, cap, D,
                                    lens.data_ptr(), 700, float("nan"), out.data_ptr(), lse.data_ptr())

        # a fresh stream has no work buffers: recording the first call is refused by name
        L.check(f.tn_stream_begin_capture(st))
        status = call()
        msg = L.last_error()
        g = ctypes.c_void_p()
        end = f.tn_stream_end_capture(st, ctypes.byref(g))
        assert status == L.TN_EINVAL and "graph capture cannot allocate" in msg, msg
        # ending that capture fails too, naming the refusal, and hands back no graph
        end_msg = L.last_error()
        assert end == L.TN_EINVAL and not g.value, (end, g.value)
        assert "refused during the capture" in end_msg and "graph capture cannot allocate" in end_msg, end_msg
        # one eager call sizes the buffers; then the same call records
        L.check(call())
        L.check(f.tn_stream_synchronize(st))
        eager_o, eager_l = out.bits(), lse.numpy()
        L.check(f.tn_stream_begin_capture(st))
        L.check(call())
        L.check(f.tn_stream_end_capture(st, ctypes.byref(g)))
        try:
            for rep in range(4):
                out.zero_()
                lse.zero_()
                tn.synchronize()
                L.check(f.tn_graph_launch(st, g.value))
                L.check(f.tn_stream_synchronize(st))
                assert np.array_equal(out.bits(), eager_o), f"replay {rep}"
                assert np.array_equal(lse.numpy(), eager_l), f"replay {rep}"
                # eager work on the same stream between the replays
                L.check(call())
                L.check(f.tn_stream_synchronize(st))
        finally:
            L.check(f.tn_graph_destroy(g.value))
    finally:
        L.check(f.tn_stream_destroy(st))
