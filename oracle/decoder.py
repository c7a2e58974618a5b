"""CPU restatement of greedy decoding with a q4_0 Llama-style decoder.

TEST INFRASTRUCTURE ONLY: the checker for tn_llama_step and the decode-step
ops. The product path never imports it.

The reference runs this model as transformers' LlamaForCausalLM on an f32
model over its torch._C ops, with every nn.Linear swapped for a Q4_0
QuantizedLinear (torchnative/python/torchnative/quant/__init__.py:100-365).
Each op below states the arithmetic it restates:

  embedding      aten.embedding.default (aten.rs:11980-12040): a row gather.
  rmsnorm        LlamaRMSNorm.forward (transformers modeling_llama.py:62-67):
                 x * rsqrt(mean(x^2) + eps) scaled by the weight; rsqrt is
                 sqrt then reciprocal (aten.rs:11112-11133).
  inv_freq/rope  LlamaRotaryEmbedding (modeling_llama.py:103-127) and
                 apply_rotary_pos_emb (:130-160): x * cos + rotate_half(x) * sin.
  silu_mul       candle's silu x / (1 + exp(-x)) (candle-core op.rs:782-784,
                 aten.rs:15360-15384) times the up projection (:174-176).
  linear         torch._C._quantized_linear: the C oracle (oracle.q4_0_linear,
                 bit-exact to the reference's x86 CPU path) in float32, or the
                 exact value of the same quantised product in float64.
  attention      the reference's default SDPA path at L=1 (oracle.sdpa).
  argmax         aten.argmax.default: first maximal index, NaN first
                 (aten.rs:11927-11975, 16705-16741).

`dtype=np.float64` runs every op except the activation quantisation in
float64; the distance between the two runs measures how sensitive the
computation itself is, which is what the GPU tolerance is scaled from.
"""

from __future__ import annotations

import numpy as np

from . import oracle as O


# the model's shape and its seeded random init are the product's own (data,
# not arithmetic), shared so that both sides decode the same model
from torchnative_amd.decoder import LlamaConfig, inv_freq, layer_weights, model_weights  # noqa: E402,F401


def rmsnorm(x, w, eps, dtype=np.float32):
    x = np.asarray(x, dtype)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=dtype)
    r = dtype(1.0) / np.sqrt(var + dtype(eps))
    return (np.asarray(w, dtype) * (x * r)).astype(dtype)


def rope(x, pos, freqs, dtype=np.float32):
    """x [..., heads, d] at position pos (scalar)."""
    x = np.asarray(x, dtype)
    half = x.shape[-1] // 2
    f = dtype(pos) * np.asarray(freqs, dtype)
    c, s = np.cos(f).astype(dtype), np.sin(f).astype(dtype)
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c + (-x2) * s, x2 * c + x1 * s], axis=-1).astype(dtype)


def silu_mul(g, u, dtype=np.float32):
    g = np.asarray(g, dtype)
    return ((g / (dtype(1.0) + np.exp(-g))) * np.asarray(u, dtype)).astype(dtype)


def argmax(x) -> int:
    x = np.asarray(x)
    nan = np.flatnonzero(np.isnan(x))
    return int(nan[0]) if nan.size else int(np.argmax(x))


def linear(x, blob, n, dtype=np.float32, threads=1):
    """Q8_0(x) . W^T for one row x [K]: the C oracle (float32), or the exact
    value of the same quantised product (float64; x is rounded to float32
    first because the activation quantiser is defined on float32)."""
    x32 = np.asarray(x, np.float32).reshape(1, -1)
    if dtype == np.float32:
        return O.q4_0_linear(x32, blob, n, threads=threads)[0]
    k = x32.shape[1]
    value, _, _ = O.exact_linear_q4_0(O.q8_0_quantize(x32), blob, 1, n, k)
    return value[0]


class Decoder:
    """The same model on the CPU, one token per step, KV cache in `dtype`."""

    def __init__(self, cfg: LlamaConfig, seed: int, cap: int, dtype=np.float32, layers=None, top=None, threads=1):
        self.cfg, self.dtype, self.cap, self.threads = cfg, dtype, cap, threads
        top = top if top is not None else model_weights(cfg, seed)
        self.embed = top["embed"]
        self.norm = top["norm"]
        self.lm_blob = O.q4_0_quantize(top["lm_head"])
        self.layers = []
        for i in range(cfg.n_layers):
            w = layers[i] if layers is not None else layer_weights(cfg, i, seed)
            self.layers.append({
                "qkv": O.q4_0_quantize(w["qkv"]), "o": O.q4_0_quantize(w["o"]),
                "gate_up": O.q4_0_quantize(w["gate_up"]), "down": O.q4_0_quantize(w["down"]),
                "ln1": w["ln1"], "ln2": w["ln2"],
                "k": np.zeros((cfg.n_kv_heads, cap, cfg.head_dim), dtype),
                "v": np.zeros((cfg.n_kv_heads, cap, cfg.head_dim), dtype),
            })
        self.freqs = inv_freq(cfg)

    def step(self, token: int, pos: int, trace=None) -> np.ndarray:
        """Process `token` at `pos`; returns the logits [vocab] in self.dtype.
        `trace`, a list, receives per layer the attention output [Hq*D] and
        the value rows the attention read [Hkv, pos+1, D]."""
        c, dt = self.cfg, self.dtype
        Hq, Hkv, D, I = c.n_heads, c.n_kv_heads, c.head_dim, c.inter
        h = self.embed[token].astype(dt)
        for L in self.layers:
            x = rmsnorm(h, L["ln1"], c.eps, dt)
            qkv = linear(x, L["qkv"], (Hq + 2 * Hkv) * D, dt, self.threads).astype(dt)
            q = rope(qkv[:Hq * D].reshape(Hq, D), pos, self.freqs, dt)
            k = rope(qkv[Hq * D:(Hq + Hkv) * D].reshape(Hkv, D), pos, self.freqs, dt)
            v = qkv[(Hq + Hkv) * D:].reshape(Hkv, D)
            L["k"][:, pos] = k
            L["v"][:, pos] = v
            a, _ = O.sdpa(q[None, :, None, :], L["k"][None, :, :pos + 1], L["v"][None, :, :pos + 1], dtype=dt)
            if trace is not None:
                trace.append({"a": a.reshape(-1).copy(), "v": L["v"][:, :pos + 1].copy()})
            h = (h + linear(a.reshape(-1), L["o"], c.hidden, dt, self.threads).astype(dt)).astype(dt)
            x = rmsnorm(h, L["ln2"], c.eps, dt)
            gu = linear(x, L["gate_up"], 2 * I, dt, self.threads).astype(dt)
            act = silu_mul(gu[:I], gu[I:], dt)
            h = (h + linear(act, L["down"], c.hidden, dt, self.threads).astype(dt)).astype(dt)
        x = rmsnorm(h, self.norm, c.eps, dt)
        return linear(x, self.lm_blob, c.vocab, dt, self.threads).astype(dt)


def linear_rows(x, blob, n, dtype=np.float32, threads=8):
    """`linear` for every row of x [T, K] at once: row-independent, so equal
    to T one-row calls (the reference's batched == one-row property,
    tests/numerics/test_qgemm.py:64-87). float32 runs the C oracle on all
    rows; float64 forms the same quantised product from the dequantised
    codes in float64 (each code times its scale is exact there; only the
    K-term sum rounds)."""
    x32 = np.ascontiguousarray(x, np.float32)
    if dtype == np.float32:
        return O.q4_0_linear(x32, blob, n, threads=threads)
    T, k = x32.shape
    xd = O.q8_0_dequantize(O.q8_0_quantize(x32), T * k).reshape(T, k).astype(np.float64)
    wd = O.q4_0_dequantize(blob, n * k).reshape(n, k).astype(np.float64)
    return xd @ wd.T


def teacher_forced_logits(dec: "Decoder", tokens, want, threads=8, trace=None) -> dict:
    """Logits of `dec`'s model at the positions in `want` when `tokens` are
    fed one per position from 0: the same values as step() called on each
    token in turn (every op is row-wise except the attention, which sees keys
    0..t for row t, i.e. upper-left causal over the sequence), computed a
    whole sequence at a time. Returns {position: logits in dec.dtype}.
    `trace`, a list, receives per layer the attention output [T, Hq*D] and
    the value rows [T, Hkv, D]."""
    c, dt = dec.cfg, dec.dtype
    Hq, Hkv, D, I = c.n_heads, c.n_kv_heads, c.head_dim, c.inter
    toks = np.asarray(tokens, np.int64)
    T = toks.size
    pos = np.arange(T)
    h = dec.embed[toks].astype(dt)
    ang = pos[:, None].astype(dt) * np.asarray(dec.freqs, dt)[None, :]
    cos, sin = np.cos(ang).astype(dt), np.sin(ang).astype(dt)

    def rope_rows(x):  # x [T, heads, D]
        half = D // 2
        x1, x2 = x[..., :half], x[..., half:]
        cc, ss = cos[:, None, :], sin[:, None, :]
        return np.concatenate([x1 * cc + (-x2) * ss, x2 * cc + x1 * ss], axis=-1).astype(dt)

    for L in dec.layers:
        x = rmsnorm(h, L["ln1"], c.eps, dt)
        qkv = linear_rows(x, L["qkv"], (Hq + 2 * Hkv) * D, dt, threads).astype(dt)
        q = rope_rows(qkv[:, :Hq * D].reshape(T, Hq, D))
        k = rope_rows(qkv[:, Hq * D:(Hq + Hkv) * D].reshape(T, Hkv, D))
        v = qkv[:, (Hq + Hkv) * D:].reshape(T, Hkv, D)
        a, _ = O.sdpa(q.transpose(1, 0, 2)[None], k.transpose(1, 0, 2)[None], v.transpose(1, 0, 2)[None],
                      is_causal=True, threads=threads, dtype=dt)
        a = a[0].transpose(1, 0, 2).reshape(T, Hq * D)
        if trace is not None:
            trace.append({"a": a.copy(), "v": v.copy()})
        h = (h + linear_rows(a, L["o"], c.hidden, dt, threads).astype(dt)).astype(dt)
        x = rmsnorm(h, L["ln2"], c.eps, dt)
        gu = linear_rows(x, L["gate_up"], 2 * I, dt, threads).astype(dt)
        act = silu_mul(gu[:, :I], gu[:, I:], dt)
        h = (h + linear_rows(act, L["down"], c.hidden, dt, threads).astype(dt)).astype(dt)
    sel = np.asarray(sorted(set(int(p) for p in want)), np.int64)
    x = rmsnorm(h[sel], dec.norm, c.eps, dt)
    logits = linear_rows(x, dec.lm_blob, c.vocab, dt, threads).astype(dt)
    return {int(p): logits[i] for i, p in enumerate(sel)}
