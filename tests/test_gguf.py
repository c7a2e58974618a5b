"""GGUF checkpoints: the container on the CPU, the loads onto the device on the GPU.

Follows the reference's tests/models/test_gguf.py: a written file reads back
(header, every metadata type, descriptors in torch order, absolute aligned
offsets); malformed files and unsupported types refuse by name; block tensors
reach the quantised tensor byte for byte; dense types read back in their own
dtype bit for bit; a GGUF linear multiplies exactly as the oracle; the Llama
q/k row permutation is undone identically on blocks and dense rows. The block
payloads include llama.cpp's own golden blobs (tests/golden/golden_gguf_py.json).
"""

import struct

import numpy as np
import pytest

import oracle as O
from gguf_write import gguf_bytes, write
from torchnative_amd import gguf as G


def _path(tmp_path, name, blob):
    p = tmp_path / name
    p.write_bytes(blob)
    return str(p)


def _rand_blocks(gtype, nblocks, seed):
    """Random GGML blocks with a finite f16 scale in each."""
    size = G.GGML_TYPES[gtype].size
    raw = np.random.default_rng(seed).integers(0, 256, size=(nblocks, size), dtype=np.uint8)
    raw[:, 1] &= 0x3B  # exponent below all-ones: finite, and |d| < 1
    if gtype == 12:
        raw[:, 3] &= 0x3B  # q4_k's dmin too
    return raw.tobytes()


# --- the container ---------------------------------------------------------------------


def test_a_written_file_reads_back_header_metadata_and_descriptors(tmp_path):
    kv = [("general.architecture", 8, "llama"), ("u8", 0, 250), ("i8", 1, -5), ("u16", 2, 65000),
          ("i16", 3, -300), ("u32", 4, 4_000_000_000), ("i32", 5, -7), ("f32", 6, 1.5), ("b", 7, True),
          ("u64", 10, 2 ** 63 + 5), ("i64", 11, -(2 ** 40)), ("f64", 12, 0.1),
          ("tokens", 9, (8, ["a", "\udcff", "ccc"])), ("ids", 9, (5, [1, -2, 3]))]
    w = _rand_blocks(2, 4, 1)
    b = np.arange(8, dtype=np.float32).tobytes()
    path = write(str(tmp_path / "a.gguf"), kv, [("w", 2, [64, 2], w), ("b", 0, [8], b)], alignment=64)
    with G.GGUFFile(path) as f:
        assert f.version == 3 and f.alignment == 64
        for key, _, v in kv:
            got = f.metadata[key]
            if isinstance(v, tuple):
                assert list(got) == v[1] and f.metadata_types[key] == (9, v[0])
            elif isinstance(v, float):
                assert got == pytest.approx(v, rel=1e-7)
            else:
                assert got == v
        assert f.metadata["tokens"][1].encode("utf-8", "surrogateescape") == b"\xff"
        wi, bi = f.info("w"), f.info("b")
        assert wi.shape == (2, 64) and wi.ne == (64, 2) and wi.type_name == "Q4_0" and wi.format == "q4_0"
        assert wi.offset % 64 == 0 and bi.offset % 64 == 0 and wi.offset >= f.data_offset
        assert bytes(f.tensor_bytes("w")) == w and bytes(f.tensor_bytes("b")) == b
        assert bi.kind == "dense" and bi.format is None and wi.nbytes == 72
        with pytest.raises(KeyError, match="no such tensor"):
            f.info("x")


@pytest.mark.parametrize("mutate,err,match", [
    (lambda b: b"GGUX" + b[4:], G.GGUFFormatError, "begins with b'GGUX'"),
    (lambda b: b[:4] + struct.pack("<I", 1) + b[8:], G.UnsupportedGGUF, "GGUF v1"),
    (lambda b: b[:4] + struct.pack(">I", 3) + b[8:], G.UnsupportedGGUF, "big-endian"),
    (lambda b: b[:4] + struct.pack("<I", 7) + b[8:], G.UnsupportedGGUF, "GGUF v7"),
    (lambda b: b[:60], G.GGUFFormatError, "the file ends inside"),
    (lambda b: b[:-10], G.GGUFFormatError, "cut short"),
    (lambda b: b[:20], G.GGUFFormatError, "shorter than the 24-byte GGUF header"),
    (lambda b: b[:8] + struct.pack("<Q", 2 ** 60) + b[16:], G.GGUFFormatError, "does not fit in"),
])
def test_malformed_files_refuse_by_name(tmp_path, mutate, err, match):
    good = gguf_bytes([("k", 4, 1)], [("w", 2, [32, 2], _rand_blocks(2, 2, 2))])
    with pytest.raises(err, match=match):
        G.GGUFFile(_path(tmp_path, "m.gguf", mutate(good)))


def test_inconsistent_descriptors_refuse_by_name(tmp_path):
    blk = _rand_blocks(2, 2, 3)
    cases = [
        (gguf_bytes([("k", 4, 1), ("k", 4, 2)], []), "duplicate metadata key 'k'"),
        (gguf_bytes([], [("w", 2, [32, 2], blk), ("w", 2, [32, 2], blk)]), "duplicate tensor name 'w'"),
        (gguf_bytes([], [("w", 2, [48, 1], blk[:27])]), "32-element blocks do not divide"),
        (gguf_bytes([], [("w", 2, [32, 2], blk)], offsets={"w": 8}), "breaks its 32-byte alignment"),
        (gguf_bytes([("general.alignment", 4, 48)], []), "must be a power of two"),
        (gguf_bytes([], [("w", 2, [], b"")]), "is 0-dimensional"),
        (gguf_bytes([], [("w", 0, [1, 1, 1, 1, 1], b"\0" * 4)]), "is 5-dimensional"),
        (gguf_bytes([("s", 9, (8, ["a"]))], [])[:24] + gguf_bytes([("s", 9, (8, ["a"]))], [])[24:41]
         + struct.pack("<Q", 2 ** 40), "says it holds 1099511627776 strings"),
        (gguf_bytes([("n", 9, (9, [(4, [1])]))], []), "array of arrays"),
    ]
    ok = gguf_bytes([("k", 4, 1)], [])  # the value type id sits after the 24-byte header and the 9-byte key
    cases.append((ok[:33] + struct.pack("<I", 13) + ok[37:], "value type 13, which GGUF does not define"))
    for i, (blob, match) in enumerate(cases):
        with pytest.raises((G.GGUFFormatError, G.UnsupportedGGUF), match=match):
            G.GGUFFile(_path(tmp_path, f"c{i}.gguf", blob))


def test_every_type_not_loaded_here_refuses_by_name(tmp_path):
    loaded = {0, 1, 2, 8, 12, 30}
    for gtype, (_, name, blk, size, kind, why) in G.GGML_TYPES.items():
        assert (gtype in loaded) == (kind != "no"), name
        if gtype in loaded:
            continue
        if blk is None:
            tensors = [("t", gtype, [32], b"")]
        else:
            tensors = [("t", gtype, [blk], b"\0" * size)]
        with G.GGUFFile(_path(tmp_path, f"t{gtype}.gguf", gguf_bytes([], tensors))) as f:
            assert f.info("t").type_name == name
            with pytest.raises(G.UnsupportedGGUF, match=f"tensor 't' is {name}, which"):
                f.tensor_bytes("t")
            with pytest.raises(G.UnsupportedGGUF):
                G.load_tensor(f, "t", keep_blocks=True, device="cpu")
            if blk is not None:
                assert bytes(f.tensor_bytes("t", allow_unloaded=True)) == b"\0" * size
    with G.GGUFFile(_path(tmp_path, "u.gguf", gguf_bytes([], [("t", 99, [4], b"")]))) as f:
        with pytest.raises(G.UnsupportedGGUF, match="GGML type id 99"):
            f.tensor_bytes("t")
    assert "activation inside a block dot" in str(G.refusal(9))
    assert "q4_0, q8_0 and q4_k blocks" in str(G.refusal(13))


def test_the_type_table_is_ggmls():
    """Block and byte sizes against the formats' own struct layouts
    (k_quants.rs:79-190 of the reference's vendored candle)."""
    qk_k = 256
    want = {"Q4_0": (32, 2 + 16), "Q8_0": (32, 2 + 32), "Q4_1": (32, 4 + 16), "Q5_0": (32, 2 + 4 + 16),
            "Q5_1": (32, 4 + 4 + 16), "Q8_1": (32, 4 + 32), "Q2_K": (qk_k, qk_k // 16 + qk_k // 4 + 4),
            "Q3_K": (qk_k, qk_k // 8 + qk_k // 4 + 12 + 2), "Q4_K": (qk_k, 4 + 12 + qk_k // 2),
            "Q5_K": (qk_k, 4 + 12 + qk_k // 8 + qk_k // 2), "Q6_K": (qk_k, qk_k // 2 + qk_k // 4 + qk_k // 16 + 2),
            "Q8_K": (qk_k, 4 + qk_k + qk_k // 16 * 2), "F32": (1, 4), "F16": (1, 2), "BF16": (1, 2)}
    byname = {v.name: v for v in G.GGML_TYPES.values()}
    for name, (blk, size) in want.items():
        assert (byname[name].block, byname[name].size) == (blk, size), name


def test_kept_blocks_stay_the_files_bytes_on_the_host(tmp_path):
    w4, w8, wk = _rand_blocks(2, 6, 4), _rand_blocks(8, 6, 5), _rand_blocks(12, 4, 6)
    path = write(str(tmp_path / "k.gguf"), [], [("a", 2, [64, 3], w4), ("b", 8, [96, 2], w8),
                                                 ("c", 12, [512, 2], wk)])
    with G.GGUFFile(path) as f:
        for name, raw, fmt in (("a", w4, "q4_0"), ("b", w8, "q8_0"), ("c", wk, "q4_k")):
            q = G.load_tensor(f, name, keep_blocks=True, device="cpu")
            assert q.format == fmt and q.shape == f.info(name).shape
            import torchnative_amd as tn
            assert tn._quantized_blob(q) == raw and tn._quantized_nbytes(q) == len(raw)


def test_qk_row_unpermutation_matches_the_dense_definition(tmp_path):
    """llama.cpp stores q/k rows interleaved per head; the loader moves whole
    rows of blocks back. Checked on the host against the dense reshape
    (n_head, dim, 2) -> (n_head, 2, dim) of the dequantised rows."""
    n_head, dim, k = 3, 4, 64
    n = n_head * 2 * dim
    raw = _rand_blocks(8, n * k // 32, 6)
    path = write(str(tmp_path / "p.gguf"), [], [("q", 8, [k, n], raw)])
    with G.GGUFFile(path) as f:
        import torchnative_amd as tn
        q = G.load_tensor(f, "q", keep_blocks=True, permute_heads=n_head, device="cpu")
        got = O.q8_0_dequantize(tn._quantized_blob(q), n * k).reshape(n, k)
        dense = O.q8_0_dequantize(raw, n * k).reshape(n, k)
        want = dense.reshape(n_head, dim, 2, k).transpose(0, 2, 1, 3).reshape(n, k)
        assert np.array_equal(got, want)
        with pytest.raises(G.UnsupportedGGUF, match="n_head=5"):
            G.load_tensor(f, "q", keep_blocks=True, permute_heads=5, device="cpu")


def test_dense_tensors_refuse_to_become_a_quantized_linear(tmp_path):
    path = write(str(tmp_path / "d.gguf"), [], [("w", 0, [32, 2], b"\0" * 256), ("v", 2, [32], b"\0" * 18)])
    with G.GGUFFile(path) as f:
        with pytest.raises(G.UnsupportedGGUF, match="needs block-quantised weights"):
            G.quantized_linear(f, "w")
        with pytest.raises(G.UnsupportedGGUF, match=r"weight is \(out_features, in_features\)"):
            G.quantized_linear(f, "v")


# --- onto the device ----------------------------------------------------------------


@pytest.fixture(scope="module")
def tn():
    import torchnative_amd as tn

    print("device:", tn._hip_probe(), flush=True)
    return tn


@pytest.mark.gpu
def test_blocks_reach_the_device_unchanged_and_dequantise_as_llama_cpp(tn, tmp_path, golden):
    cases, _ = golden
    tensors, want = [], {}
    for (fmt, name), c in sorted(cases.items()):
        if fmt not in ("q4_0", "q8_0"):
            continue
        shape = c["shape"] if len(c["shape"]) == 2 else [1, c["shape"][0]]
        tensors.append((f"{fmt}.{name}", 2 if fmt == "q4_0" else 8, shape[::-1], bytes.fromhex(c["blob"])))
        want[f"{fmt}.{name}"] = (bytes.fromhex(c["blob"]), bytes.fromhex(c["dequant_f32"]))
    tensors.append(("rand4", 2, [256, 40], _rand_blocks(2, 320, 7)))
    tensors.append(("rand8", 8, [128, 33], _rand_blocks(8, 132, 8)))
    tensors.append(("rand4k", 12, [512, 6], _rand_blocks(12, 12, 9)))
    path = write(str(tmp_path / "g.gguf"), [], tensors)
    with G.GGUFFile(path) as f:
        for name, gtype, _, raw in tensors:
            q = G.load_tensor(f, name, keep_blocks=True)
            assert q.device == "hip" and tn._quantized_blob(q) == raw, name
            dq = G.load_tensor(f, name).numpy().reshape(-1).tobytes()
            deq = {2: O.q4_0_dequantize, 8: O.q8_0_dequantize, 12: O.q4_k_dequantize}[gtype]
            assert dq == deq(raw, f.info(name).n_elements).tobytes(), name
            if name in want:
                assert dq == want[name][1], name


@pytest.mark.gpu
def test_dense_types_read_back_exactly_in_their_own_dtype(tn, tmp_path):
    rng = np.random.default_rng(9)
    f32 = rng.standard_normal((5, 7)).astype(np.float32)
    f16 = rng.standard_normal((3, 8)).astype(np.float16)
    bf = rng.integers(0, 0x7F00, size=(4, 6), dtype=np.uint16)
    path = write(str(tmp_path / "d.gguf"), [], [("a", 0, [7, 5], f32.tobytes()), ("b", 1, [8, 3], f16.tobytes()),
                                                 ("c", 30, [6, 4], bf.tobytes())])
    with G.GGUFFile(path) as f:
        a, b, c = (G.load_tensor(f, n) for n in "abc")
        assert (a.dtype, b.dtype, c.dtype) == ("float32", "float16", "bfloat16")
        assert a.bits().tobytes() == f32.tobytes() and b.bits().tobytes() == f16.tobytes()
        assert c.bits().tobytes() == bf.tobytes() and c.shape == (4, 6)


@pytest.mark.gpu
@pytest.mark.parametrize("gtype", [2, 8, 12])
def test_a_gguf_linear_holds_the_file_bytes_and_multiplies_as_the_oracle(tn, tmp_path, gtype):
    n, k = 96, 512
    raw = {2: lambda: O.synth_q4_0_weight(n, k, 0.02, 10), 8: lambda: O.synth_q8_0_weight(n, k, 0.02, 10),
           12: lambda: O.synth_q4_k_weight(n, k, 10)}[gtype]()
    bias = np.random.default_rng(11).standard_normal(n).astype(np.float32)
    path = write(str(tmp_path / "l.gguf"), [], [("blk.0.ffn_down.weight", gtype, [k, n], raw)])
    x = np.random.default_rng(12).standard_normal((3, k)).astype(np.float32)
    lin_fn = {2: O.q4_0_linear, 8: O.q8_0_linear, 12: O.q4_k_linear}[gtype]
    with G.GGUFFile(path) as f:
        lin = G.quantized_linear(f, "blk.0.ffn_down.weight", bias=tn.tensor(bias, device="hip"))
    assert (lin.out_features, lin.in_features) == (n, k)
    assert tn._quantized_blob(lin.qweight) == raw
    for m in (1, 3):
        got = lin(tn.tensor(x[:m], device="hip")).numpy()
        assert got.tobytes() == lin_fn(x[:m], raw, n, bias=bias).tobytes()
