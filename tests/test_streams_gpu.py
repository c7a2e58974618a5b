"""Work on two streams at once. Each stream keeps its own workspace and
ticket counters (runtime.hip), so calls enqueued on two streams and left to
overlap must give the same bits as the same calls made one at a time. The
cases are the paths that use a workspace or tickets: the f32 stream-K
prefill (cut query blocks merged through tickets), the bf16 prefill at head
dim 128 (split rows merged through tickets), the stream-K decode and its
combine, and the q4 GEMM with its activation prepass. Two rounds swap which
stream runs which half, and every output has its own buffer.
"""

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


def _cases(tn):
    from torchnative_amd import _lib as L

    lib = L.lib()
    rng = np.random.default_rng(7)
    dev = lambda a, dt: tn.tensor(a.astype(np.float32), dtype=dt, device="hip")
    cases = []

    def prefill(dt, B, Hq, Hkv, S, D, causal):
        q = dev(rng.standard_normal((B, Hq, S, D)), dt)
        k = dev(rng.standard_normal((B, Hkv, S, D)), dt)
        v = dev(rng.standard_normal((B, Hkv, S, D)), dt)
        code = {"float32": L.TN_F32, "bfloat16": L.TN_BF16}[dt]

        def alloc():
            return tn.empty((B, Hq, S, D), dt, "hip"), tn.empty((B, Hq, S), "float32", "hip")

        def launch(stream, outs):
            out, lse = outs
            L.check(lib.tn_sdpa_fwd(stream, code, q.data_ptr(), k.data_ptr(), v.data_ptr(), B, Hq, Hkv, S, S, D,
                                    None, 0, None, causal, float("nan"), out.data_ptr(), lse.data_ptr()))

        return alloc, launch

    def decode(B, Hq, Hkv, D, cap):
        q = dev(rng.standard_normal((B, Hq, D)), "bfloat16")
        k = dev(rng.standard_normal((B, Hkv, cap, D)), "bfloat16")
        v = dev(rng.standard_normal((B, Hkv, cap, D)), "bfloat16")
        lens = rng.integers(1, cap + 1, B).astype(np.int32)
        ln = tn.tensor(lens, device="hip")

        def alloc():
            return tn.empty((B, Hq, D), "bfloat16", "hip"), tn.empty((B, Hq), "float32", "hip")

        def launch(stream, outs):
            out, lse = outs
            L.check(lib.tn_sdpa_decode(stream, L.TN_BF16, q.data_ptr(), k.data_ptr(), v.data_ptr(), B, Hq, Hkv, cap,
                                       D, ln.data_ptr(), int(lens.max()), float("nan"), out.data_ptr(),
                                       lse.data_ptr()))

        return alloc, launch

    def gemm(m, k, n):
        blob = O.synth_q4_0_weight(n, k, 0.02, 3)
        w = tn._quantized_from_blob(blob, (n, k), "q4_0", device="hip")
        x = tn.tensor(rng.standard_normal((m, k)).astype(np.float32), device="hip")

        def alloc():
            return (tn.empty((m, n), "float32", "hip"),)

        def launch(stream, outs):
            L.check(lib.tn_q4_0_linear(stream, x.data_ptr(), L.TN_F32, m, k, *w._planes(), n, None,
                                       outs[0].data_ptr(), L.TN_F32))

        return alloc, launch

    cases.append(("f32 prefill", prefill("float32", 1, 8, 2, 1536, 64, 1)))
    cases.append(("bf16 prefill d128", prefill("bfloat16", 1, 8, 2, 2048, 128, 1)))
    cases.append(("decode", decode(8, 16, 4, 128, 2048)))
    cases.append(("q4 gemm", gemm(64, 2048, 1024)))
    return cases


def test_two_streams_overlapping_give_the_same_bits(tn):
    s1, s2 = tn.Stream(), tn.Stream()
    cases = _cases(tn)
    tn.synchronize()
    want = {}
    for name, (alloc, launch) in cases:  # one at a time, each finished before the next
        outs = alloc()
        launch(s1.handle, outs)
        s1.synchronize()
        want[name] = [t.bits() for t in outs]
    for rnd in range(2):
        outs = {name: alloc() for name, (alloc, _) in cases}  # every buffer exists before the first launch
        tn.synchronize()
        for i, (name, (_, launch)) in enumerate(cases):  # alternate streams; nothing waits in between
            launch((s1, s2)[(i + rnd) % 2].handle, outs[name])
        s1.synchronize()
        s2.synchronize()
        for name, _ in cases:
            for j, (a, b) in enumerate(zip(want[name], outs[name])):
                assert np.array_equal(a, b.bits()), f"round {rnd}: {name} output {j} differs"
