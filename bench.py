"""Benchmark of the hot path on one MI355X (the BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

One step is one pass of the hot path over one batch of synthetic input, with
the inputs already resident in HBM. The headline line is BASELINE config 2
(causal GQA SDPA prefill, bf16, B=1, 9/3 heads, D=64, S=2048); the other
configs are measured in the same run and reported under "parts":

  c1  q4_0 decode GEMV [1,576] x [1536,576]^T, streamed over 1,024 distinct
      weight copies in one launch (509 MB > the 256 MB MALL), plus the latency
      of one C1-sized call;
  c2  SDPA prefill, bf16 (headline) and fp32;
  c3  q4_0 prefill GEMM x bf16 [512,4096] x W [14336,4096]^T, bf16 out;
  c4  decode attention, B=16, 32/8 heads, D=128, bf16, lens ~ U[512,4096],
      rotated over 3 KV sets (> MALL);
  c5  greedy decode of the random-init 30-layer q4_0 Llama, 256-token prompt,
      128 new tokens, tokens/s over the steps after the prompt.

Kernel time comes from HIP events on the stream the kernels run on; the
step time from the host clock around synchronised regions. The CPU baseline
is the C oracle (the restatement of the reference's CPU arithmetic) timed on
this host's cores on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
INT8_PEAK_TOPS = 5000.0

# weight format -> (GGML bytes per block, device code bytes per block, elements per block)
_BLOCK = {"q4_0": (18, 16, 32), "q8_0": (34, 32, 32), "q4_k": (144, 144, 256)}


def _synth_q4_0_blob(n, k, sigma, seed):
    """Q4_0 blob in the BASELINE format: codes uniform in [-8,7] (nib = code+8),
    d = f16_rne(|N(0, sigma)| / 7)."""
    rng = np.random.default_rng(seed)
    nb = k // 32
    nib = rng.integers(0, 16, size=(n, nb, 32), dtype=np.uint8)
    d = (np.abs(rng.standard_normal((n, nb))) * sigma / 7.0).astype(np.float32).astype(np.float16)
    blob = np.empty((n, nb, 18), dtype=np.uint8)
    blob[:, :, 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    blob[:, :, 2:] = nib[:, :, :16] | (nib[:, :, 16:] << 4)
    return blob.reshape(-1)


def _synth_q8_0_blob(n, k, sigma, seed):
    """Q8_0 blob: codes uniform in [-127, 127], d = f16_rne(|N(0, sigma)| / 127)."""
    rng = np.random.default_rng(seed)
    nb = k // 32
    codes = rng.integers(-127, 128, size=(n, nb, 32), dtype=np.int8)
    d = (np.abs(rng.standard_normal((n, nb))) * sigma / 127.0).astype(np.float32).astype(np.float16)
    blob = np.empty((n, nb, 34), dtype=np.uint8)
    blob[:, :, 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    blob[:, :, 2:] = codes.view(np.uint8)
    return blob.reshape(-1)


def _synth_q4_k_blob(n, k, sigma, seed):
    """Q4_K blob: random nibbles and 6-bit scales/mins, d = f16(|N(0, sigma)|/63),
    dmin = f16(|N(0, sigma/10)|/63)."""
    rng = np.random.default_rng(seed)
    nb = k // 256
    blob = rng.integers(0, 256, size=(n, nb, 144), dtype=np.uint8)
    d = (np.abs(rng.standard_normal((n, nb))) * sigma / 63).astype(np.float32).astype(np.float16)
    dm = (np.abs(rng.standard_normal((n, nb))) * sigma / 630).astype(np.float32).astype(np.float16)
    blob[:, :, 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    blob[:, :, 2:4] = dm.view(np.uint8).reshape(n, nb, 2)
    return blob.reshape(-1)


def _synth_blob(fmt, n, k, sigma, seed):
    return {"q8_0": _synth_q8_0_blob, "q4_0": _synth_q4_0_blob, "q4_k": _synth_q4_k_blob}[fmt](n, k, sigma, seed)


class Timer:
    """Host wall clock around a synchronised region plus HIP events on the
    stream the work is issued to."""

    def __init__(self, tn, stream=None):
        self.tn, self.stream = tn, stream
        self.e0, self.e1 = tn.Event(), tn.Event()

    def run(self, fn, steps, warmup):
        for _ in range(warmup):
            fn()
        self.tn.synchronize()
        t0 = time.perf_counter()
        self.e0.record(self.stream)
        for _ in range(steps):
            fn()
        self.e1.record(self.stream)
        self.tn.synchronize()
        wall = (time.perf_counter() - t0) * 1e3
        return wall / steps, self.e0.elapsed_ms(self.e1) / steps


def bench_sdpa(tn, L, dtype, steps, warmup, B=1, Hq=9, Hkv=3, S=2048, D=64, seed=2):
    rng = np.random.default_rng(seed)
    q = tn.tensor(rng.standard_normal((B, Hq, S, D)).astype(np.float32), dtype=dtype, device="hip")
    k = tn.tensor(rng.standard_normal((B, Hkv, S, D)).astype(np.float32), dtype=dtype, device="hip")
    v = tn.tensor(rng.standard_normal((B, Hkv, S, D)).astype(np.float32), dtype=dtype, device="hip")
    out = tn.empty((B, Hq, S, D), dtype, "hip")
    lse = tn.empty((B, Hq, S), "float32", "hip")
    code = L.TN_BF16 if dtype == "bfloat16" else L.TN_F32
    lib = L.lib()

    def step():
        st = lib.tn_sdpa_fwd(None, code, q.data_ptr(), k.data_ptr(), v.data_ptr(), B, Hq, Hkv, S, S, D, None, 0, None, 1,
                             float("nan"), out.data_ptr(), lse.data_ptr())
        if st:
            L.check(st)

    ms, kern_ms = Timer(tn).run(step, steps, warmup)
    flops = 4.0 * D * Hq * B * S * (S + 1) / 2
    peak = BF16_PEAK_TFLOPS if dtype == "bfloat16" else FP32_PEAK_TFLOPS
    ach = flops / (kern_ms * 1e-3) / 1e12
    return {"ms_per_step": ms, "kernel_ms": kern_ms, "flops": flops, "tflops": flops / (ms * 1e-3) / 1e12,
            "roofline": {"bound": "mfma", "achieved": ach, "peak": peak, "unit": "TFLOP/s", "frac": ach / peak,
                         "traffic": None}}


def bench_sdpa_masked(tn, L, steps, warmup, B=1, Hq=9, Hkv=3, S=2048, D=64, pad=64, seed=2):
    """Config 2's shape (bf16, causal, GQA) with a bool padding mask
    [B, 1, 1, S] that hides the last `pad` keys, as a padded batch passes
    to F.scaled_dot_product_attention. A mask that is the same for every
    query row runs on the kernel without split rows (k_fa64), which stages
    each ring stage's mask values in LDS. flops = 4 D Hq over the (query,
    key) pairs both the causal rule and the mask let through."""
    rng = np.random.default_rng(seed)
    q = tn.tensor(rng.standard_normal((B, Hq, S, D)).astype(np.float32), dtype="bfloat16", device="hip")
    k = tn.tensor(rng.standard_normal((B, Hkv, S, D)).astype(np.float32), dtype="bfloat16", device="hip")
    v = tn.tensor(rng.standard_normal((B, Hkv, S, D)).astype(np.float32), dtype="bfloat16", device="hip")
    keep = np.ones((B, 1, 1, S), np.bool_)
    keep[..., S - pad:] = False
    mask = tn.tensor(keep, device="hip")
    strides = (ctypes.c_int64 * 4)(S, 0, 0, 1)  # element strides over (B, Hq, L, S): broadcast heads and rows
    out = tn.empty((B, Hq, S, D), "bfloat16", "hip")
    lse = tn.empty((B, Hq, S), "float32", "hip")
    lib = L.lib()

    def step():
        st = lib.tn_sdpa_fwd(None, L.TN_BF16, q.data_ptr(), k.data_ptr(), v.data_ptr(), B, Hq, Hkv, S, S, D,
                             mask.data_ptr(), L.TN_BOOL, strides, 1, float("nan"), out.data_ptr(), lse.data_ptr())
        if st:
            L.check(st)

    ms, kern_ms = Timer(tn).run(step, steps, warmup)
    valid = S - pad
    # row i attends keys 0 .. min(i, valid - 1)
    pairs = sum(min(i, valid - 1) + 1 for i in range(S))
    flops = 4.0 * D * Hq * B * pairs
    ach = flops / (kern_ms * 1e-3) / 1e12
    return {"ms_per_step": ms, "kernel_ms": kern_ms, "flops": flops, "tflops": flops / (ms * 1e-3) / 1e12,
            "mask": f"bool [B,1,1,S], last {pad} keys hidden", "kernel": "k_fa64",
            "roofline": {"bound": "mfma", "achieved": ach, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": ach / BF16_PEAK_TFLOPS, "traffic": None}}


def bench_gemv(tn, L, steps, warmup, copies=1024, fmt="q4_0"):
    # q4_k needs K % 256 == 0: its leg uses K = 768 (C1's 576 rounded up)
    n, k = 1536, (768 if fmt == "q4_k" else 576)
    lib = L.lib()
    blob_b, code_b, blk = _BLOCK[fmt]
    from_blob, linear = getattr(lib, f"tn_{fmt}_from_blob"), getattr(lib, f"tn_{fmt}_linear")
    planes = (lambda q, d: (q,)) if fmt == "q4_k" else (lambda q, d: (q, d))
    rng = np.random.default_rng(1)
    x = tn.tensor(rng.standard_normal((1, k)).astype(np.float32), device="hip")
    # 1,024 distinct [1536, 576] weights, contiguous: one launch streams all of them
    qs = tn.empty((copies * n * k // blk * code_b,), "uint8", "hip")
    dd = tn.empty((copies * n * k // blk * 2,), "uint8", "hip")
    chunk = 64
    for c0 in range(0, copies, chunk):
        blob = _synth_blob(fmt, chunk * n, k, 0.02, 1000 + c0)
        bt = tn.tensor(blob, device="hip")
        off_q = c0 * n * k // blk * code_b
        off_d = c0 * n * k // blk * 2
        L.check(from_blob(None, bt.data_ptr(), chunk * n, k, *planes(qs.data_ptr() + off_q, dd.data_ptr() + off_d)))
    y = tn.empty((1, copies * n), "float32", "hip")

    def step_all():
        st = linear(None, x.data_ptr(), L.TN_F32, 1, k, *planes(qs.data_ptr(), dd.data_ptr()), copies * n, None,
                    y.data_ptr(), L.TN_F32)
        if st:
            L.check(st)

    # C1 is the first GPU work of a run: a longer warm-up (about 10 ms) lets
    # the clocks settle before the timed region
    ms, kern_ms = Timer(tn).run(step_all, steps, max(warmup, 100))
    w_bytes = n * (k // blk) * blob_b
    per_copy = w_bytes + n * 4
    total_bytes = copies * per_copy + k * 4
    ach = total_bytes / (kern_ms * 1e-3) / 1e9
    # one C1-sized call, cycling through the copies so the weight is cold
    idx = [0]

    def step_one():
        c = idx[0] % copies
        idx[0] += 1
        st = linear(None, x.data_ptr(), L.TN_F32, 1, k,
                    *planes(qs.data_ptr() + c * n * k // blk * code_b, dd.data_ptr() + c * n * k // blk * 2), n,
                    None, y.data_ptr(), L.TN_F32)
        if st:
            L.check(st)

    one_ms, one_kern = Timer(tn).run(step_one, max(steps, 50), warmup)
    return {"ms_per_step": ms, "kernel_ms": kern_ms, "copies": copies, "bytes_per_launch": total_bytes,
            "algorithmic_bytes_per_c1_call": w_bytes + k * 4 + n * 4, "gbs": total_bytes / (ms * 1e-3) / 1e9,
            "single_call_us": one_kern * 1e3,
            "single_call_gbs": (w_bytes + k * 4 + n * 4) / (one_kern * 1e-3) / 1e9,
            "roofline": {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": ach / HBM_PEAK_GBS, "traffic": None}}


def bench_gemm(tn, L, steps, warmup, fmt="q4_0"):
    m, k, n = 512, 4096, 14336
    lib = L.lib()
    linear = getattr(lib, f"tn_{fmt}_linear")
    rng = np.random.default_rng(3)
    x = tn.tensor(rng.standard_normal((m, k)).astype(np.float32), dtype="bfloat16", device="hip")
    q = tn._quantized_from_blob(_synth_blob(fmt, n, k, 0.01, 33).tobytes(), (n, k), fmt, device="hip")
    y = tn.empty((m, n), "bfloat16", "hip")

    def step():
        st = linear(None, x.data_ptr(), L.TN_BF16, m, k, *q._planes(), n, None,
                                y.data_ptr(), L.TN_BF16)
        if st:
            L.check(st)

    ms, kern_ms = Timer(tn).run(step, steps, warmup)
    flops = 2.0 * m * k * n
    ach = flops / (kern_ms * 1e-3) / 1e12
    # the block dots run on bf16 MFMA for q4_0 and on int8 MFMA for q8_0; q4_k
    # is priced against the bf16 peak
    peak, unit = (INT8_PEAK_TOPS, "TOP/s") if fmt == "q8_0" else (BF16_PEAK_TFLOPS, "TFLOP/s")
    return {"ms_per_step": ms, "kernel_ms": kern_ms, "flops": flops, "tflops": flops / (ms * 1e-3) / 1e12,
            "bytes": n * (k // _BLOCK[fmt][2]) * _BLOCK[fmt][0] + m * k * 2 + m * n * 2,
            "roofline": {"bound": "mfma", "achieved": ach, "peak": peak, "unit": unit,
                         "frac": ach / peak, "traffic": None}}


def bench_decode(tn, L, steps, warmup, sets=3):
    B, Hq, Hkv, D, cap = 16, 32, 8, 128, 4096
    lib = L.lib()
    rng = np.random.default_rng(4)
    lens_np = rng.integers(512, 4097, size=B).astype(np.int32)
    lens = tn.tensor(lens_np, device="hip")
    max_len = int(lens_np.max())
    q = tn.tensor(rng.standard_normal((B, Hq, D)).astype(np.float32), dtype="bfloat16", device="hip")
    caches = []
    for s in range(sets):
        kc = tn.empty((B, Hkv, cap, D), "bfloat16", "hip")
        vc = tn.empty((B, Hkv, cap, D), "bfloat16", "hip")
        for t in (kc, vc):
            bits = tn.tensor(rng.standard_normal((B * Hkv * cap * D // 8,)).astype(np.float32), dtype="bfloat16",
                             device="hip")
            # fill with N(0,1) bf16 (8 repeats of a random block keep host memory small)
            for r in range(8):
                L.check(lib.tn_memcpy_d2d(t.data_ptr() + r * bits.nbytes, bits.data_ptr(), bits.nbytes, None))
        caches.append((kc, vc))
    out = tn.empty((B, Hq, D), "bfloat16", "hip")
    lse = tn.empty((B, Hq), "float32", "hip")
    idx = [0]

    def step():
        kc, vc = caches[idx[0] % sets]
        idx[0] += 1
        st = lib.tn_sdpa_decode(None, L.TN_BF16, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), B, Hq, Hkv, cap, D,
                                lens.data_ptr(), max_len, float("nan"), out.data_ptr(), lse.data_ptr())
        if st:
            L.check(st)

    ms, kern_ms = Timer(tn).run(step, steps, warmup)
    kv_bytes = int(lens_np.sum()) * Hkv * D * 2 * 2
    total = kv_bytes + 2 * B * Hq * D * 2
    ach = total / (kern_ms * 1e-3) / 1e9
    return {"ms_per_step": ms, "kernel_ms": kern_ms, "bytes": total, "gbs": total / (ms * 1e-3) / 1e9,
            "lens_sum": int(lens_np.sum()),
            "roofline": {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": ach / HBM_PEAK_GBS, "traffic": None}}


def bench_e2e(tn, L, prompt_len=256, n_new=128, seed=5, graph=True):
    """greedy decode of the random-init 30-layer q4_0
    Llama (hidden 576, 9/3 heads, MLP 1536, vocab 49152). As the reference's
    bench does (tests/bench/bench_llama_cpp.py:540-569), the prompt yields
    the first token and the next n_new - 1 steps are timed: tokens/s =
    (n_new - 1) / seconds. The timed steps run as one captured HIP graph;
    the same steps issued one call at a time are reported beside it. The
    prompt runs as one batched prefill (tn_llama_prefill), timed on its own
    as the reference's bench times its prefill phase
    (tests/bench/bench_llama_cpp.py:484-523): prefill tokens/s = prompt
    tokens / seconds, at the 256-token prompt and at 128 tokens."""
    from torchnative_amd.decoder import LlamaConfig, Q4Llama

    cfg = LlamaConfig()
    model = Q4Llama(cfg, seed=0, cap=prompt_len + n_new)
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab, prompt_len).astype(np.int32)
    s = ctypes.c_void_p()
    L.check(L.lib().tn_stream_create(ctypes.byref(s)))
    st = s.value
    lib = L.lib()

    def run_prompt():
        model.start(prompt)
        model.prefill(prompt_len, st)
        L.check(lib.tn_stream_synchronize(st))

    def time_prefill(n, reps=7):
        model.start(prompt[:n])
        model.prefill(n, st)  # warm: the GEMM workspace, first-touch
        L.check(lib.tn_stream_synchronize(st))
        ts = []
        for _ in range(reps):
            model.start(prompt[:n])
            L.check(lib.tn_stream_synchronize(st))
            t0 = time.perf_counter()
            model.prefill(n, st)
            L.check(lib.tn_stream_synchronize(st))
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    graph_s = tokens = warm_tokens = None
    try:
        prefill_s = {n: time_prefill(n) for n in (128, prompt_len)}
        # the stepwise prompt's first tokens, beside the batched prompt's
        model.start(prompt)
        for _ in range(prompt_len):
            model.step(st)
        for _ in range(15):
            model.step(st)
        L.check(lib.tn_stream_synchronize(st))
        stepwise_tokens = model.generated(prompt_len, 16)
        if graph:
            run_prompt()
            g = model.capture(n_new - 1, st)
            g.launch(st)  # warm: the first launch uploads the graph
            L.check(lib.tn_stream_synchronize(st))
            warm_tokens = model.generated(prompt_len, n_new)
            run_prompt()
            t0 = time.perf_counter()
            g.launch(st)
            L.check(lib.tn_stream_synchronize(st))
            graph_s = time.perf_counter() - t0
            tokens = model.generated(prompt_len, n_new)
            g.close()
        run_prompt()
        t0 = time.perf_counter()
        for _ in range(n_new - 1):
            model.step(st)
        L.check(lib.tn_stream_synchronize(st))
        eager_s = time.perf_counter() - t0
        eager_tokens = model.generated(prompt_len, n_new)
    finally:
        L.check(lib.tn_stream_destroy(st))
    weight_bytes = cfg.n_layers * ((cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim * cfg.hidden
                                   + cfg.hidden * cfg.n_heads * cfg.head_dim + 3 * cfg.inter * cfg.hidden)
    weight_bytes = (weight_bytes + cfg.vocab * cfg.hidden) // 32 * 18
    timed_s = graph_s if graph else eager_s
    tps = (n_new - 1) / timed_s
    return {"tokens_per_s": tps, "ms_per_token": timed_s * 1e3 / (n_new - 1), "graph": graph,
            "eager_tokens_per_s": (n_new - 1) / eager_s, "prompt_tokens": prompt_len, "new_tokens": n_new,
            "prefill": {"tokens_per_s": prompt_len / prefill_s[prompt_len], "ms": prefill_s[prompt_len] * 1e3,
                        "tokens_per_s_128": 128 / prefill_s[128], "ms_128": prefill_s[128] * 1e3,
                        "method": "tn_llama_prefill, host wall clock around a synchronised call, median of 7",
                        "reference_published": {"tokens_per_s": {"128": 220.6, "512": 210.3},
                                                "hardware": "Apple M1 CPU, 4 threads, SmolLM2-135M q4_0"}},
            "first_tokens_stepwise_prompt": stepwise_tokens,
            "q4_weight_bytes_per_token": weight_bytes,
            "weight_stream_gbs": weight_bytes * tps / 1e9,
            "same_tokens_graph_eager_warm": (tokens == eager_tokens == warm_tokens) if graph else None,
            "first_tokens": (tokens if graph else eager_tokens)[:16]}


def host_cpu():
    """The host's CPU model, physical cores (distinct (package, core id)
    pairs) and logical CPUs this process may use."""
    model, cores, pkg = None, set(), None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = (s.strip() for s in line.partition(":"))
                if key == "model name" and model is None:
                    model = val
                elif key == "physical id":
                    pkg = val
                elif key == "core id":
                    cores.add((pkg, val))
    except OSError:
        pass
    logical = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"cpu_model": model, "physical_cores": len(cores) or None, "logical_cpus": logical}


def cpu_threads():
    """Threads for the CPU baselines: the reference's default is one per
    physical core (candle-core/src/utils.rs:312-323); on a shared GPU box the
    process's CPU share (OMP_NUM_THREADS, 16 there) caps it."""
    h = host_cpu()
    n = min(h["physical_cores"] or h["logical_cpus"], h["logical_cpus"])
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, min(n, share) if share > 0 else n)


def _timed(fn, seconds):
    fn()  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        sec = time.perf_counter() - t0
        if sec >= seconds:
            return reps, sec


def _cpu_record(value, unit, threads, sample, **extra):
    return {"value": value, "unit": unit, "cores": threads, "kind": "port", "sample": sample, **host_cpu(), **extra}


def cpu_baseline_q4(threads, m, seconds, c1=True):
    """The oracle's bit-exact restatement of the reference's x86 CPU q4_0
    linear (Q8_0 activations, scalar vec_dot_unopt, the 4-column driver:
    k_quants.rs:312-329, :2430-2582) on the config-1 shape (GB/s of the same
    algorithmic bytes as the GPU line) or on m rows of the config-3 shape
    (TFLOP/s of 2 m k n)."""
    import oracle as O

    if c1:
        n, k = 1536, 576
        blob = _synth_q4_0_blob(n, k, 0.02, 1).tobytes()
        x = np.random.default_rng(1).standard_normal((1, k)).astype(np.float32)
    else:
        n, k = 14336, 4096
        blob = _synth_q4_0_blob(n, k, 0.01, 33).tobytes()
        x = O.bf16_to_f32(O.bf16_from_f32(np.random.default_rng(3).standard_normal((m, k)).astype(np.float32)))
    reps, sec = _timed(lambda: O.q4_0_linear(x, blob, n, threads=threads), seconds)
    if c1:
        nbytes = n * k // 32 * 18 + k * 4 + n * 4
        return _cpu_record(nbytes * reps / sec / 1e9, "GB/s", threads,
                           f"config 1 in full ([1,576] x [1536,576]^T q4_0) x {reps} calls in {sec:.1f} s",
                           us_per_call=sec / reps * 1e6)
    flops = 2.0 * m * k * n
    return _cpu_record(flops * reps / sec / 1e12, "TFLOP/s", threads,
                       f"{m} of config 3's 512 rows ([{m},4096] x [14336,4096]^T q4_0, bf16 x widened) x {reps} "
                       f"calls in {sec:.1f} s; a full config-3 call would take {sec / reps * 512 / m:.2f} s")


def cpu_baseline_decode(threads, seconds):
    """The oracle's default SDPA path at L=1 per sequence over the config-4
    caches (B=16, 32/8 heads, D=128, bf16 widened to f32, the same lengths as
    the GPU run), in GB/s of the same K/V bytes."""
    import oracle as O

    B, Hq, Hkv, D = 16, 32, 8, 128
    rng = np.random.default_rng(4)
    lens = rng.integers(512, 4097, size=B)
    q = O.bf16_to_f32(O.bf16_from_f32(rng.standard_normal((B, Hq, D)).astype(np.float32)))
    kv = [O.bf16_to_f32(O.bf16_from_f32(rng.standard_normal((2, Hkv, int(n), D)).astype(np.float32))) for n in lens]

    def call():
        for b in range(B):
            O.bf16_from_f32(O.sdpa(q[b][None, :, None, :], kv[b][0][None], kv[b][1][None], threads=threads)[0])

    reps, sec = _timed(call, seconds)
    nbytes = int(lens.sum()) * Hkv * D * 2 * 2 + 2 * B * Hq * D * 2
    return _cpu_record(nbytes * reps / sec / 1e9, "GB/s", threads,
                       f"config 4 in full (16 sequences, lengths as the GPU run, sum {int(lens.sum())}) x {reps} "
                       f"calls in {sec:.1f} s", us_per_call=sec / reps * 1e6)


def cpu_baseline_e2e(threads, steps=12, start=256):
    """The oracle's float32 decode step of the config-5 model (the C q4_0
    linear bit-exact to the reference's x86 path, numpy for the rest) at
    positions 256.. with the KV cache filled with random values, in tokens/s.
    For context, the reference publishes 86.4 tok/s for SmolLM2-135M q4_0 on
    an Apple M1 CPU with 4 threads (tests/bench/results_llama_cpp.json)."""
    from oracle import decoder as OD

    cfg = OD.LlamaConfig()
    dec = OD.Decoder(cfg, 0, start + steps + 1, np.float32, threads=threads)
    rng = np.random.default_rng(7)
    for L in dec.layers:
        L["k"][:] = rng.standard_normal(L["k"].shape).astype(np.float32)
        L["v"][:] = rng.standard_normal(L["v"].shape).astype(np.float32)
    tok = 17
    dec.step(tok, start)  # warm
    t0 = time.perf_counter()
    for i in range(steps):
        tok = OD.argmax(dec.step(tok, start + 1 + i))
    sec = time.perf_counter() - t0
    return _cpu_record(steps / sec, "tokens/s", threads,
                       f"{steps} greedy steps of the config-5 model at positions {start + 1}..{start + steps} "
                       f"(KV cache pre-filled), {sec:.1f} s",
                       reference_published={"value": 86.4, "unit": "tokens/s",
                                            "hardware": "Apple M1 CPU, 4 threads, SmolLM2-135M q4_0",
                                            "source": "tests/bench/results_llama_cpp.json"})


def cpu_baseline_sdpa(threads, seconds=10.0):
    """The oracle's restatement of the reference's default SDPA path (f32
    body, bf16 in/out) on the full config 2 (9/3 heads, causal, S=2048),
    repeated until about `seconds` of wall time have passed, in TFLOP/s of the
    same algorithmic flop count as the GPU line. The oracle's products are
    plain triple loops, so this understates the reference's default path,
    whose two products run in the gemm crate with runtime SIMD dispatch."""
    import oracle as O

    rng = np.random.default_rng(2)
    S, D, hq, hkv = 2048, 64, 9, 3
    q = O.bf16_to_f32(O.bf16_from_f32(rng.standard_normal((1, hq, S, D)).astype(np.float32)))
    k = O.bf16_to_f32(O.bf16_from_f32(rng.standard_normal((1, hkv, S, D)).astype(np.float32)))
    v = O.bf16_to_f32(O.bf16_from_f32(rng.standard_normal((1, hkv, S, D)).astype(np.float32)))
    O.sdpa(q[:, :, :64], k, v, is_causal=True, threads=threads)  # warm
    reps = 0
    t0 = time.perf_counter()
    while True:
        out, _ = O.sdpa(q, k, v, is_causal=True, threads=threads)
        O.bf16_from_f32(out)
        reps += 1
        sec = time.perf_counter() - t0
        if sec >= seconds:
            break
    flops = 4.0 * D * hq * S * (S + 1) / 2 * reps
    return _cpu_record(flops / sec / 1e12, "TFLOP/s", threads,
                       f"config 2 in full (9 q heads / 3 kv heads, causal, S=2048, bf16 inputs widened to f32, "
                       f"output narrowed to bf16) x {reps} repetitions: {sec:.1f} s for {flops / 1e9:.1f} GFLOP; "
                       "scalar loops for the two products, so below the reference's gemm-crate default path")


# The copy kernel that scales the PMC byte counters: tn_q4_0_from_blob over a
# 288 MiB blob reads and writes each of its bytes exactly once.
COPY_CAL_BLOCKS = 16 * 1024 * 1024


def calibrate_copy(tn, L, steps):
    lib = L.lib()
    nbytes = COPY_CAL_BLOCKS * 18
    blob = tn.empty((nbytes,), "uint8", "hip")
    blob.zero_()
    qs = tn.empty((COPY_CAL_BLOCKS * 16,), "uint8", "hip")
    d = tn.empty((COPY_CAL_BLOCKS,), "float16", "hip")  # the f16 scale plane
    for _ in range(steps):
        L.check(lib.tn_q4_0_from_blob(None, blob.data_ptr(), COPY_CAL_BLOCKS, 32, qs.data_ptr(), d.data_ptr()))
    tn.synchronize()
    print(json.dumps({"copy_kernel": "tn_q4_0_from_blob", "read_bytes": nbytes, "write_bytes": nbytes,
                      "launches": steps}))


def profiled_traffic(name):
    """HBM bytes per launch of a config's dominant kernel, as committed in
    profiles/<name> (line `traffic_bytes_per_launch: N`), or None."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default="", help="comma list of parts to run (c1,c2,c2f32,c2mask,c3,c4,c5,q8c1,q8c3,q4kc1,q4kc3)")
    ap.add_argument("--no-graph", action="store_true",
                    help="c5: time the decode steps as separate launches only (no HIP graph)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only the copy kernel that scales rocprofv3's FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} asked); the path would shard by "
              "KV-head group for SDPA and by output columns for the q4 linear, with no collective on the path. "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torchnative_amd as tn
    from torchnative_amd import _lib as L

    info = tn._hip_probe()
    if args.calibrate_copy:
        calibrate_copy(tn, L, args.steps)
        return
    only = set(filter(None, args.only.split(",")))
    want = (lambda p: not only or p in only)
    parts = {}
    if want("c1"):
        print("bench: c1 q4_0 GEMV", file=sys.stderr, flush=True)
        parts["c1_q4_gemv"] = bench_gemv(tn, L, args.steps, args.warmup)
    if want("c2f32"):
        print("bench: c2 SDPA prefill fp32", file=sys.stderr, flush=True)
        parts["c2_sdpa_prefill_fp32"] = bench_sdpa(tn, L, "float32", args.steps, args.warmup)
    if want("c2mask"):
        print("bench: c2 SDPA prefill bf16 with a bool padding mask", file=sys.stderr, flush=True)
        parts["c2_sdpa_prefill_bf16_padding_mask"] = bench_sdpa_masked(tn, L, args.steps, args.warmup)
    if want("c3"):
        print("bench: c3 q4_0 GEMM", file=sys.stderr, flush=True)
        parts["c3_q4_gemm"] = bench_gemm(tn, L, args.steps, args.warmup)
    if want("q8c1"):
        print("bench: q8_0 GEMV at the c1 shape", file=sys.stderr, flush=True)
        parts["q8_0_gemv_c1_shape"] = bench_gemv(tn, L, args.steps, args.warmup, fmt="q8_0")
    if want("q8c3"):
        print("bench: q8_0 GEMM at the c3 shape", file=sys.stderr, flush=True)
        parts["q8_0_gemm_c3_shape"] = bench_gemm(tn, L, args.steps, args.warmup, fmt="q8_0")
    if want("q4kc1"):
        print("bench: q4_k GEMV at the c1 shape (K 768)", file=sys.stderr, flush=True)
        parts["q4_k_gemv_c1_shape"] = bench_gemv(tn, L, args.steps, args.warmup, fmt="q4_k")
    if want("q4kc3"):
        print("bench: q4_k prefill at the c3 shape", file=sys.stderr, flush=True)
        parts["q4_k_gemm_c3_shape"] = bench_gemm(tn, L, args.steps, args.warmup, fmt="q4_k")
    if want("c4"):
        print("bench: c4 decode attention", file=sys.stderr, flush=True)
        parts["c4_decode_attention"] = bench_decode(tn, L, args.steps, args.warmup)
    if want("c5"):
        print("bench: c5 end-to-end greedy decode", file=sys.stderr, flush=True)
        parts["c5_e2e_decode"] = bench_e2e(tn, L, graph=not args.no_graph)
    print("bench: c2 SDPA prefill bf16 (headline)", file=sys.stderr, flush=True)
    head = bench_sdpa(tn, L, "bfloat16", args.steps, args.warmup)
    head["roofline"]["traffic"] = profiled_traffic("flash_bf16_c2_traffic.md")
    # the parts' dominant kernels, measured the same way (rocprofv3 FETCH_SIZE
    # and WRITE_SIZE passes scaled by the copy calibration)
    for part, prof in (("c1_q4_gemv", "q4_gemv_c1.md"), ("c2_sdpa_prefill_fp32", "flash_f32_c2.md"),
                       ("c3_q4_gemm", "q4_gemm_c3.md"), ("c4_decode_attention", "decode_attention_c4.md")):
        if part in parts:
            parts[part]["roofline"]["traffic"] = profiled_traffic(prof)

    cpu = None
    if not args.no_cpu_baseline:
        th = cpu_threads()
        print(f"bench: cpu baselines ({th} threads)", file=sys.stderr, flush=True)
        cpu = cpu_baseline_sdpa(th, seconds=8.0)
        legs = {"c1_q4_gemv": lambda: cpu_baseline_q4(th, 1, 3.0),
                "c3_q4_gemm": lambda: cpu_baseline_q4(th, 16, 4.0, c1=False),
                "c4_decode_attention": lambda: cpu_baseline_decode(th, 3.0),
                "c5_e2e_decode": lambda: cpu_baseline_e2e(th)}
        for name, fn in legs.items():
            if name in parts:
                parts[name]["cpu_baseline"] = fn()
        if "c2_sdpa_prefill_fp32" in parts:
            parts["c2_sdpa_prefill_fp32"]["cpu_baseline"] = cpu

    line = {
        "metric": "q4 GEMV HBM GB/s + SDPA TFLOP/s (% roofline); decode tokens/s, 1 GPU",
        "value": head["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "BASELINE config 2: causal GQA SDPA prefill, B=1, 9 q heads / 3 kv heads, "
                               "head_dim 64, seq 2048, bf16 in/out, f32 accumulate",
                   "flops_per_step": head["flops"]},
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "device": info.get("name") or info.get("arch"),
        "parts": parts,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
