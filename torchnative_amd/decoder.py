"""Greedy decoding of a q4_0 Llama-style decoder on the hip device.

the reference runs this as transformers'
LlamaForCausalLM on an f32 model with every nn.Linear swapped for a Q4_0
QuantizedLinear (torchnative/python/torchnative/quant/__init__.py:100-365)
and greedy `generate` (tests/bench/bench_llama_cpp.py:540-569). Here the
whole step runs on the device through `tn_llama_step` (include/tnhip.h):
the embedding, RMSNorm, rotary embedding, the q4_0 linears, the f32 decode
attention over a preallocated KV cache, the SiLU-gated MLP, the residual
adds and the argmax. The step keeps its position and token on the device,
so the prompt and the generated tokens run as one sequence of identical
steps that `capture` can record as a HIP graph.

A prompt runs either one token per step, or in one batched pass per layer
(`prefill`, `tn_llama_prefill`: the q4_0 linears as GEMMs over the prompt's
rows and the causal f32 prefill attention), after which the steps continue.
The q4_0 linear of a row does not depend on how many rows are batched with
it, so both give the reference's prefill values up to the attention's
summation order.
"""

from __future__ import annotations

import ctypes
import zlib
from dataclasses import dataclass

import numpy as np

from . import _C, _lib
from ._lib import check, lib
from .tensor import Tensor, current_stream


@dataclass(frozen=True)
class LlamaConfig:
    """BASELINE config 5's model by default (SmolLM2-135M's shape)."""

    n_layers: int = 30
    hidden: int = 576
    n_heads: int = 9
    n_kv_heads: int = 3
    head_dim: int = 64
    inter: int = 1536
    vocab: int = 49152
    eps: float = 1e-5
    rope_theta: float = 1e5


def init_weight(name: str, shape, seed: int, std: float = 0.02) -> np.ndarray:
    """Deterministic random-init f32 weight N(0, std), seeded by the weight's
    name (transformers initialises linears and embeddings with N(0, 0.02))."""
    rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
    return (rng.standard_normal(shape) * std).astype(np.float32)


def layer_weights(cfg: LlamaConfig, layer: int, seed: int) -> dict:
    """One decoder layer's f32 weights, the projections stacked as the step
    runs them (q|k|v rows, gate|up rows); norm weights are ones."""
    H, D, I = cfg.hidden, cfg.head_dim, cfg.inter
    p = f"layers.{layer}."
    qkv = np.concatenate([init_weight(p + "q_proj", (cfg.n_heads * D, H), seed),
                          init_weight(p + "k_proj", (cfg.n_kv_heads * D, H), seed),
                          init_weight(p + "v_proj", (cfg.n_kv_heads * D, H), seed)], axis=0)
    gate_up = np.concatenate([init_weight(p + "gate_proj", (I, H), seed),
                              init_weight(p + "up_proj", (I, H), seed)], axis=0)
    return {"qkv": qkv, "o": init_weight(p + "o_proj", (H, cfg.n_heads * D), seed), "gate_up": gate_up,
            "down": init_weight(p + "down_proj", (H, I), seed),
            "ln1": np.ones(H, np.float32), "ln2": np.ones(H, np.float32)}


def model_weights(cfg: LlamaConfig, seed: int) -> dict:
    return {"embed": init_weight("embed_tokens", (cfg.vocab, cfg.hidden), seed),
            "norm": np.ones(cfg.hidden, np.float32),
            "lm_head": init_weight("lm_head", (cfg.vocab, cfg.hidden), seed)}


def inv_freq(cfg: LlamaConfig) -> np.ndarray:
    """1 / theta^(arange(0, d, 2) / d) in float32, as LlamaRotaryEmbedding
    computes it (modeling_llama.py compute_default_rope_parameters)."""
    d = cfg.head_dim
    e = (np.arange(0, d, 2, dtype=np.float32) / np.float32(d)).astype(np.float32)
    return (np.float32(1.0) / np.power(np.float32(cfg.rope_theta), e, dtype=np.float32)).astype(np.float32)


class Q4Llama:
    """The model resident on the device: q4_0 weight planes (quantised on the
    device from f32, bit-exact to the reference's quantize_), f32 embedding
    and norms, an f32 KV cache of `cap` positions per layer."""

    def __init__(self, cfg: LlamaConfig = LlamaConfig(), seed: int = 0, cap: int = 512, weights=None):
        """weights: None for the seeded random init, else a callable
        layer -> dict and a dict for the embedding/norm/lm_head, as
        (layer_fn, top)."""
        self.cfg, self.cap = cfg, int(cap)
        layer_fn, top = weights if weights is not None else (
            (lambda i: layer_weights(cfg, i, seed)), model_weights(cfg, seed))
        keep = []  # device tensors the descriptor points at

        def dev(a, dtype=None):
            t = Tensor.from_numpy(a, dtype=dtype, device="hip")
            keep.append(t)
            return t

        staging = []  # f32 uploads, released after the quantiser has run

        def q4(w):
            f = Tensor.from_numpy(w, device="hip")
            staging.append(f)
            qt = _C._quantize(f, "q4_0")
            keep.extend([qt._qs, qt._d])
            return _lib.Q4Weight(qt._qs.data_ptr(), qt._d.data_ptr())

        def release():
            check(lib().tn_stream_synchronize(current_stream()))
            staging.clear()

        D, Hkv = cfg.head_dim, cfg.n_kv_heads
        self._layers = (_lib.LlamaLayer * cfg.n_layers)()
        for i in range(cfg.n_layers):
            w = layer_fn(i)
            L = self._layers[i]
            L.qkv, L.o, L.gate_up, L.down = q4(w["qkv"]), q4(w["o"]), q4(w["gate_up"]), q4(w["down"])
            L.ln1, L.ln2 = dev(w["ln1"]).data_ptr(), dev(w["ln2"]).data_ptr()
            kc = Tensor((Hkv, self.cap, D), "float32", "hip").zero_()
            vc = Tensor((Hkv, self.cap, D), "float32", "hip").zero_()
            keep.extend([kc, vc])
            L.k_cache, L.v_cache = kc.data_ptr(), vc.data_ptr()
            release()
        m = _lib.Llama()
        m.n_layers, m.hidden, m.n_heads, m.n_kv_heads = cfg.n_layers, cfg.hidden, cfg.n_heads, cfg.n_kv_heads
        m.head_dim, m.inter, m.vocab, m.cap, m.eps = cfg.head_dim, cfg.inter, cfg.vocab, self.cap, cfg.eps
        m.embed = dev(top["embed"]).data_ptr()
        m.norm = dev(top["norm"]).data_ptr()
        m.lm_head = q4(top["lm_head"])
        m.inv_freq = dev(inv_freq(cfg)).data_ptr()
        release()
        m.layers = ctypes.cast(self._layers, ctypes.POINTER(_lib.LlamaLayer))
        self.state = Tensor((4,), "int32", "hip").zero_()
        self.tokens = Tensor((self.cap,), "int32", "hip").zero_()
        self.logits = Tensor((cfg.vocab,), "float32", "hip")
        m.state, m.tokens, m.logits = self.state.data_ptr(), self.tokens.data_ptr(), self.logits.data_ptr()
        # one prompt buffer for the model's life: a captured graph holds its address
        self._prompt = Tensor((self.cap,), "int32", "hip").zero_()
        m.prompt, m.prompt_len = self._prompt.data_ptr(), 0
        self._desc = m
        self.work = Tensor((int(lib().tn_llama_work_floats(ctypes.byref(m))),), "float32", "hip")
        m.work = self.work.data_ptr()
        self._keep = keep
        self._prefill_work = None
        self._prefill_tokens = 0

    # --- running -----------------------------------------------------------------------
    def start(self, prompt_ids) -> None:
        """Load a prompt and rewind to position 0 (the caches need no
        clearing: a step reads positions below its own only)."""
        ids = np.asarray(prompt_ids, dtype=np.int32).reshape(-1)
        if ids.size < 1 or ids.size > self.cap:
            raise ValueError(f"prompt of {ids.size} tokens does not fit a cache of {self.cap}")
        if ids.min() < 0 or ids.max() >= self.cfg.vocab:
            raise ValueError("prompt token id outside the vocabulary")
        check(lib().tn_memcpy_h2d(self._prompt.data_ptr(), ids.ctypes.data, ids.nbytes, current_stream()))
        self._desc.prompt_len = int(ids.size)
        st = np.array([0, 1, ids[0], 0], dtype=np.int32)
        check(lib().tn_memcpy_h2d(self.state.data_ptr(), st.ctypes.data, st.nbytes, current_stream()))
        check(lib().tn_memcpy_h2d(self.tokens.data_ptr(), ids.ctypes.data, 4, current_stream()))

    def step(self, stream=None) -> None:
        check(lib().tn_llama_step(stream if stream is not None else current_stream(), ctypes.byref(self._desc)))

    def prefill(self, tokens=None, stream=None) -> None:
        """Run the loaded prompt's first `tokens` (all of it by default) in one
        batched pass; the next step() continues at position `tokens`."""
        t = int(self._desc.prompt_len if tokens is None else tokens)
        if self._prefill_work is None or self._prefill_tokens < t:
            n = int(lib().tn_llama_prefill_work_floats(ctypes.byref(self._desc), t))
            self._prefill_work = Tensor((n,), "float32", "hip")
            self._prefill_tokens = t
        check(lib().tn_llama_prefill(stream if stream is not None else current_stream(), ctypes.byref(self._desc), t,
                                     self._prefill_work.data_ptr()))

    def capture(self, steps: int, stream) -> "Graph":
        """Record `steps` consecutive steps as one HIP graph on `stream` (a
        created stream). The graph reads the step state from the device, so
        it can be replayed from any position."""
        g = ctypes.c_void_p()
        check(lib().tn_llama_capture(stream, ctypes.byref(self._desc), int(steps), ctypes.byref(g)))
        return Graph(g.value, self)

    def position(self) -> int:
        return int(self.state.numpy()[0])

    def generated(self, n_prompt: int, n_new: int) -> list:
        """The n_new tokens after an n_prompt-token prompt."""
        return [int(t) for t in self.tokens.numpy()[n_prompt:n_prompt + n_new]]

    def generate(self, prompt_ids, max_new_tokens: int, stream=None, graph: bool = False,
                 prefill: bool = False) -> list:
        """Greedy decoding: the prompt's last position yields the first new
        token, each further step one more (max_new_tokens - 1 steps after the
        prompt). prefill: the prompt in one batched pass instead of a step
        per token."""
        n = len(prompt_ids)
        if n + max_new_tokens - 1 > self.cap:
            raise ValueError(f"{n} prompt + {max_new_tokens} new tokens do not fit a cache of {self.cap}")
        self.start(prompt_ids)
        if prefill:
            self.prefill(n, stream)
        else:
            for _ in range(n):
                self.step(stream)
        rest = max_new_tokens - 1
        if rest > 0:
            if graph:
                g = self.capture(rest, stream)
                g.launch(stream)
                g.close()
            else:
                for _ in range(rest):
                    self.step(stream)
        check(lib().tn_stream_synchronize(stream if stream is not None else current_stream()))
        return self.generated(n, max_new_tokens)


class Graph:
    """A captured run of decode steps (hipGraphExec_t)."""

    def __init__(self, handle, owner):
        self.handle, self._owner = handle, owner

    def launch(self, stream) -> None:
        check(lib().tn_graph_launch(stream, self.handle))

    def close(self) -> None:
        if self.handle:
            check(lib().tn_graph_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
