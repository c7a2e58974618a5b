"""BASELINE config 5's model at its real size on the MI355X, against the oracle.

30 layers, hidden 576, 9 query / 3 key-value heads of 64, SiLU MLP 1536,
RMSNorm 1e-5, RoPE theta 1e5, vocab 49152, every linear (lm_head included)
q4_0 -- the model the bench decodes. It is fed a 384-token sequence one token
per step (teacher-forced: every position gets the same token on both sides)
and its logits are compared at positions 0-7, 255-262, 300-303 and 380-383
(the bench's timed steps are positions 256-383 of a 384-entry cache) with the
oracle's float32 run (oracle/decoder.py, the reference's x86 q4 linear bit for
bit and its default SDPA path), computed a whole sequence at a time.

Bound: oracle.sdpa_tolerance per position, i.e. 4x the oracle's own
float32-vs-float64 distance on the same tokens, floored at 1.186e-6 of the
logits' scale. The float64 run quantises its activations to Q8_0 too, so
that distance includes the activation-code flips a last-bit difference can
cause, which the GPU's different summation orders cause as well. The greedy
token (the step's argmax) must be the oracle's wherever the oracle's top two
logits are further apart than twice the bound.

Both attention paths of the step: cap 384 runs the fused split attention
(12 splits of 32 keys, merged in the o projection's prologue), cap 600 the
RoPE + append kernel, the split-KV decode attention and its combine.
"""

import numpy as np
import pytest

import oracle as O
from oracle import decoder as OD

pytestmark = pytest.mark.gpu

SEED = 20
N_TOK = 384
WANT = list(range(8)) + list(range(255, 263)) + list(range(300, 304)) + list(range(380, 384))


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


@pytest.fixture(scope="module")
def c5():
    """The weights (generated once), the token sequence and the oracle's
    float32 / float64 logits at the wanted positions."""
    cfg = OD.LlamaConfig()
    layers = [OD.layer_weights(cfg, i, SEED) for i in range(cfg.n_layers)]
    top = OD.model_weights(cfg, SEED)
    toks = np.random.default_rng(SEED).integers(0, cfg.vocab, N_TOK).astype(np.int32)
    print("c5: oracle float32 run", flush=True)
    r32 = OD.teacher_forced_logits(OD.Decoder(cfg, SEED, N_TOK, np.float32, layers, top), toks, WANT, threads=16)
    print("c5: oracle float64 run", flush=True)
    r64 = OD.teacher_forced_logits(OD.Decoder(cfg, SEED, N_TOK, np.float64, layers, top), toks, WANT, threads=16)
    return cfg, layers, top, toks, r32, r64


@pytest.mark.parametrize("cap", [384, 600])
def test_config5_model_teacher_forced_against_the_oracle(tn, c5, cap):
    from torchnative_amd.decoder import Q4Llama

    cfg, layers, top, toks, r32, r64 = c5
    print(f"c5: cap {cap}, building the model on the device", flush=True)
    model = Q4Llama(cfg, seed=SEED, cap=cap, weights=(lambda i: layers[i], top))
    model.start(toks)  # the whole sequence as the prompt: every step gets the given token
    worst, checked_tokens = 0.0, 0
    for pos in range(N_TOK):
        model.step()
        if pos not in r32:
            continue
        got = model.logits.numpy().astype(np.float64)
        l32, l64 = r32[pos].astype(np.float64), r64[pos]
        tol = O.sdpa_tolerance(l32, l64, "float32")
        w = float(np.max(np.abs(got - l32) / tol))
        worst = max(worst, w)
        assert w <= 1.0, f"cap {cap} position {pos}: {w:.3g}x the bound"
        top2 = np.sort(l32)[-2:]
        if top2[1] - top2[0] > 2 * float(np.max(tol)):
            assert int(model.state.numpy()[3]) == OD.argmax(l32), f"cap {cap} position {pos}: greedy token"
            checked_tokens += 1
    print(f"c5: cap {cap}: worst {worst:.3f} of the bound, greedy token checked at {checked_tokens} positions",
          flush=True)


# The fused split attention across several 32-key splits with a fresh row in
# a later split, at config 5's head shape (head_dim 64, 3 query heads per kv
# head) on a small model: a 150-token prompt crosses several split
# boundaries, and cap 200 keeps the fused path (7 splits).
NREP3 = OD.LlamaConfig(n_layers=2, hidden=384, n_heads=6, n_kv_heads=2, head_dim=64, inter=256, vocab=512)


@pytest.mark.parametrize("cap", [200, 512])
def test_fused_split_attention_across_split_boundaries(tn, cap):
    from torchnative_amd.decoder import Q4Llama

    rng = np.random.default_rng(cap)
    prompt = [int(t) for t in rng.integers(0, NREP3.vocab, 150)]
    n_new = 12
    model = Q4Llama(NREP3, seed=13, cap=cap)
    r32 = OD.Decoder(NREP3, 13, cap, np.float32)
    r64 = OD.Decoder(NREP3, 13, cap, np.float64)
    model.start(prompt)
    seq = list(prompt)
    for pos in range(len(prompt) + n_new - 1):
        model.step()
        l32 = r32.step(seq[pos], pos).astype(np.float64)
        l64 = r64.step(seq[pos], pos)
        if pos >= 60:  # from just below the first split boundary on
            tol = O.sdpa_tolerance(l32, l64, "float32")
            w = float(np.max(np.abs(model.logits.numpy() - l32) / tol))
            assert w <= 1.0, f"cap {cap} position {pos}: {w:.3g}x the bound"
        nxt = int(model.state.numpy()[2])
        if pos + 1 >= len(prompt):
            seq.append(nxt)
    assert model.generated(len(prompt), n_new) == seq[len(prompt):]


# The decoder's composition on the device, with weights that make the answer
# known (the oracle's composition is pinned the same way on the CPU,
# tests/test_oracle_decoder.py): every o and down projection zero, so the
# logits are lm_head(rmsnorm(embed[t])) at every position; the q and k rows
# zero, so every head attends uniformly to positions 0..t of its key/value
# head h // 3. Both on the cap-200 fused split attention and the cap-600
# split-KV path, over 150 teacher-forced tokens.
GQA3 = OD.LlamaConfig(n_layers=3, hidden=384, n_heads=6, n_kv_heads=2, head_dim=64, inter=256, vocab=512)


def _zeroed(cfg, seed, *, qk=False, o_down=False):
    D = cfg.head_dim
    layers = []
    for i in range(cfg.n_layers):
        w = dict(OD.layer_weights(cfg, i, seed))
        if qk:
            w["qkv"] = w["qkv"].copy()
            w["qkv"][:(cfg.n_heads + cfg.n_kv_heads) * D] = 0.0
        if o_down:
            w["o"] = np.zeros_like(w["o"])
            w["down"] = np.zeros_like(w["down"])
        layers.append(w)
    return layers, OD.model_weights(cfg, seed)


@pytest.mark.parametrize("cap", [200, 600])
@pytest.mark.parametrize("which", ["o_down", "qk"])
def test_decoder_composition_with_zeroed_projections(tn, cap, which):
    from torchnative_amd.decoder import Q4Llama

    layers, top = _zeroed(GQA3, 31, qk=which == "qk", o_down=which == "o_down")
    toks = np.random.default_rng(cap).integers(0, GQA3.vocab, 150).astype(np.int32)
    want = list(range(0, 150, 7)) + [149]
    r32 = OD.teacher_forced_logits(OD.Decoder(GQA3, 31, 150, np.float32, layers, top), toks, want)
    r64 = OD.teacher_forced_logits(OD.Decoder(GQA3, 31, 150, np.float64, layers, top), toks, want)
    model = Q4Llama(GQA3, seed=31, cap=cap, weights=(lambda i: layers[i], top))
    model.start(toks)
    lm = O.q4_0_quantize(top["lm_head"])
    for pos in range(len(toks)):
        model.step()
        if pos not in r32:
            continue
        got = model.logits.numpy().astype(np.float64)
        l32, l64 = r32[pos].astype(np.float64), r64[pos]
        tol = O.sdpa_tolerance(l32, l64, "float32")
        w = float(np.max(np.abs(got - l32) / tol))
        assert w <= 1.0, f"{which} cap {cap} position {pos}: {w:.3g}x the bound"
        if which == "o_down":
            # the closed form itself: the oracle's logits are exactly it (CPU test), the device's within the bound
            x = OD.rmsnorm(top["embed"][int(toks[pos])], top["norm"], GQA3.eps)
            closed = O.q4_0_linear(x.reshape(1, -1), lm, GQA3.vocab)[0].astype(np.float64)
            assert np.array_equal(closed, l32)


# The prompt in one batched pass (tn_llama_prefill: the q4_0 GEMM over the
# prompt's rows, the causal f32 prefill attention), then decode steps from
# there: the last prompt position's logits and the later steps' against the
# same oracle run as the step-by-step test above, on both attention paths of
# the steps that follow.
@pytest.mark.parametrize("cap", [384, 600])
def test_config5_batched_prefill_then_steps_against_the_oracle(tn, c5, cap):
    from torchnative_amd.decoder import Q4Llama

    cfg, layers, top, toks, r32, r64 = c5
    model = Q4Llama(cfg, seed=SEED, cap=cap, weights=(lambda i: layers[i], top))
    model.start(toks)  # teacher-forced: the sequence is the prompt; the first 256 run batched
    T = 256
    model.prefill(T)
    assert model.position() == T  # the state advanced past the batched positions
    assert np.array_equal(model.tokens.numpy()[:T + 1], toks[:T + 1])
    worst = 0.0

    def check(pos):
        nonlocal worst
        got = model.logits.numpy().astype(np.float64)
        l32, l64 = r32[pos].astype(np.float64), r64[pos]
        tol = O.sdpa_tolerance(l32, l64, "float32")
        w = float(np.max(np.abs(got - l32) / tol))
        worst = max(worst, w)
        assert w <= 1.0, f"cap {cap} position {pos}: {w:.3g}x the bound"
        top2 = np.sort(l32)[-2:]
        if top2[1] - top2[0] > 2 * float(np.max(tol)):
            assert int(model.state.numpy()[3]) == OD.argmax(l32), f"cap {cap} position {pos}: greedy token"

    check(T - 1)  # the prefill's own logits
    for pos in range(T, N_TOK):
        model.step()
        if pos in r32:
            check(pos)
    print(f"c5 prefill: cap {cap}: worst {worst:.3f} of the bound", flush=True)


# head dim 48: a head's rows are not whole 32-element Q8_0 blocks, so the
# prompt's o projection reads the attention output through the copy to
# token rows instead of in place
HD48 = OD.LlamaConfig(n_layers=2, hidden=288, n_heads=6, n_kv_heads=2, head_dim=48, inter=256, vocab=512)


@pytest.mark.parametrize("cfg,n_prompt", [(NREP3, 1), (NREP3, 5), (NREP3, 64), (NREP3, 150), (HD48, 5), (HD48, 70)],
                         ids=["hd64-1", "hd64-5", "hd64-64", "hd64-150", "hd48-5", "hd48-70"])
def test_prefill_generates_the_oracles_greedy_tokens(tn, cfg, n_prompt):
    """A small model: prefill a prompt of n tokens and generate 12 more with
    the steps; every generated token is the oracle's greedy token wherever
    the oracle's top two logits are further apart than twice the bound."""
    from torchnative_amd.decoder import Q4Llama

    rng = np.random.default_rng(n_prompt)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab, n_prompt)]
    n_new = 12
    model = Q4Llama(cfg, seed=13, cap=200)
    got = model.generate(prompt, n_new, prefill=True)
    r32 = OD.Decoder(cfg, 13, 200, np.float32)
    r64 = OD.Decoder(cfg, 13, 200, np.float64)
    seq = list(prompt)
    for pos in range(n_prompt + n_new - 1):
        l32 = r32.step(seq[pos], pos).astype(np.float64)
        l64 = r64.step(seq[pos], pos)
        if pos + 1 >= n_prompt:
            i = pos + 1 - n_prompt
            tol = O.sdpa_tolerance(l32, l64, "float32")
            top2 = np.sort(l32)[-2:]
            if top2[1] - top2[0] > 2 * float(np.max(tol)):
                assert got[i] == OD.argmax(l32), f"prompt {n_prompt}: new token {i}"
            seq.append(got[i])
