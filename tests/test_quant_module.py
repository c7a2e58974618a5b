"""`quantize_`, `QuantizedLinear` and `.to()` (the reference's
torchnative/python/torchnative/quant/__init__.py:100-365) over a model tree.

On the CPU: the tree walk, the refusals of a bare Linear and of a model with
nothing to replace, and the predicate. On the GPU: every Linear is swapped,
lm_head included; a layer whose in_features is not a multiple of the block
size stays dense and is reported with the quantiser's reason; the report's
bytes are the dense and GGML sizes; a swapped layer computes exactly what
`_quantized_linear` over `_quantize(W)` plus the bias computes (the oracle's
bits); and `.to("cpu")` / `.to("hip")` move the blocks byte for byte.
"""

import numpy as np
import pytest

import oracle as O
from torchnative_amd import nn
from torchnative_amd.quant import QuantizedLinear, quantize_


class Block(nn.Module):
    def __init__(self, rng, device):
        super().__init__()
        self.q_proj = nn.Linear(rng.standard_normal((64, 64)) * 0.02, device=device)
        self.up = nn.Linear(rng.standard_normal((96, 64)) * 0.02, rng.standard_normal(96), device=device)
        self.odd = nn.Linear(rng.standard_normal((10, 48)) * 0.02, device=device)  # 48 % 32 != 0


class Model(nn.Module):
    def __init__(self, device="cpu", seed=0):
        super().__init__()
        rng = np.random.default_rng(seed)
        self.layers = nn.ModuleList([Block(rng, device), Block(rng, device)])
        self.norm_scale = 1.0  # not a module
        self.lm_head = nn.Linear(rng.standard_normal((128, 64)) * 0.02, device=device)


def test_the_walk_sees_every_linear_with_its_dotted_name():
    names = [n for n, m in Model().named_modules() if isinstance(m, nn.Linear)]
    assert names == ["layers.0.q_proj", "layers.0.up", "layers.0.odd", "layers.1.q_proj", "layers.1.up",
                     "layers.1.odd", "lm_head"]


def test_a_bare_linear_and_an_empty_model_are_refused():
    with pytest.raises(ValueError, match="bare Linear"):
        quantize_(nn.Linear(np.zeros((4, 32)), device="cpu"))
    with pytest.raises(ValueError, match="holds no Linear"):
        quantize_(nn.Module())


def test_a_predicate_that_excludes_everything_reports_every_layer():
    m = Model()
    rep = quantize_(m, "q4_0", predicate=lambda name, mod: False)
    assert rep.replaced == [] and len(rep.skipped) == 7
    assert set(rep.reasons()) == {"excluded by the predicate"}
    assert isinstance(m.lm_head, nn.Linear)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_every_linear_is_swapped_lm_head_included_and_computes_the_oracles_bits(fmt):
    import torchnative_amd as tn

    dense = Model(device="cpu", seed=3)
    weights = {n: (m.weight.numpy(), None if m.bias is None else m.bias.numpy())
               for n, m in dense.named_modules() if isinstance(m, nn.Linear)}
    model = Model(device="hip", seed=3)
    rep = quantize_(model, fmt)
    # parents are visited in tree order, so the root's own lm_head comes first
    assert rep.replaced == ["lm_head", "layers.0.q_proj", "layers.0.up", "layers.1.q_proj", "layers.1.up"]
    assert [n for n, _ in rep.skipped] == ["layers.0.odd", "layers.1.odd"]
    assert all("not a multiple of 32" in why for _, why in rep.skipped)
    assert isinstance(model.lm_head, QuantizedLinear) and isinstance(model.layers[0].odd, nn.Linear)
    per = {"q4_0": 18, "q8_0": 34}[fmt]
    numel = sum(weights[n][0].size for n in rep.replaced)
    assert rep.dense_bytes == 4 * numel and rep.quantized_bytes == numel // 32 * per
    assert f"{len(rep.replaced)} layers replaced, 2 skipped" in str(rep) and "layers.0.odd" in str(rep)
    quantize = O.q4_0_quantize if fmt == "q4_0" else O.q8_0_quantize
    linear = O.q4_0_linear if fmt == "q4_0" else O.q8_0_linear
    x = np.random.default_rng(4).standard_normal((3, 64)).astype(np.float32)
    for name in rep.replaced:
        layer = dict(model.named_modules())[name]
        w, b = weights[name]
        assert tn._quantized_blob(layer.qweight) == quantize(w)
        got = layer(tn.tensor(x, device="hip")).numpy()
        assert got.tobytes() == linear(x, quantize(w), w.shape[0], bias=b).tobytes(), name


@pytest.mark.gpu
def test_to_moves_the_blocks_byte_for_byte_and_back():
    import torchnative_amd as tn

    model = Model(device="hip", seed=5)
    quantize_(model, "q4_0")
    blobs = {n: tn._quantized_blob(m.qweight) for n, m in model.named_modules() if isinstance(m, QuantizedLinear)}
    x = tn.tensor(np.random.default_rng(6).standard_normal((2, 64)).astype(np.float32), device="hip")
    before = model.layers[1].up(x).numpy()
    model.to("cpu")
    for n, m in model.named_modules():
        if isinstance(m, QuantizedLinear):
            assert m.device == "cpu" and tn._quantized_blob(m.qweight) == blobs[n]
            if m.bias is not None:
                assert m.bias.device == "cpu"
    assert model.layers[0].odd.weight.device == "cpu"  # the dense layer moved too
    with pytest.raises(RuntimeError, match="Expected all tensors to be on the same device"):
        model.lm_head(x)  # the reference's message for a hip input and a cpu weight (quant.rs:313-320)
    model.to("hip")
    for n, m in model.named_modules():
        if isinstance(m, QuantizedLinear):
            assert m.device == "hip" and tn._quantized_blob(m.qweight) == blobs[n]
    assert np.array_equal(model.layers[1].up(x).numpy(), before)
