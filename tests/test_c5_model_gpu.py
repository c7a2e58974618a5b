"""BASELINE config 5's model at its real size on the MI355X, against the oracle.

30 layers, hidden 576, 9 query / 3 key-value heads of 64, SiLU MLP 1536,
RMSNorm 1e-5, RoPE theta 1e5, vocab 49152, every linear (lm_head included)
q4_0 -- the model the bench decodes. It is fed a 263-token sequence one token
per step (teacher-forced: every position gets the same token on both sides)
and its logits are compared at positions 0-7 and 255-262 with the oracle's
float32 run (oracle/decoder.py, the reference's x86 q4 linear bit for bit and
its default SDPA path), computed a whole sequence at a time.

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
N_TOK = 263
WANT = list(range(8)) + list(range(255, 263))


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
