"""Writes tests/golden/q4_k_writer.json: Q4_K writer input/output vectors.

Nothing stored in the reference pins the Q4_K writer's bytes: its own test
(tests/numerics/test_q4kwriter.py) computes the expected bytes at test time
from a scalar transcription of llama.cpp's quantize_row_q4_K_ref
(ggml-quants.c at 3de52ac3, lines 630-635, 808-896, 1467-1535), on fixtures
it builds in `_fixtures()`. This script runs that transcription once, in the
development container where the reference checkout exists, and stores its
inputs and outputs as data. Only the transcription's own functions and
constants are taken from the file (its test-harness imports are not needed
for them). The reference does not travel: the JSON holds float32 inputs and
the blob bytes, both as hex.

Run: python3 tests/golden/make_q4_k_writer_vectors.py [path/to/reference]
"""

import ast
import json
import math
import os
import struct
import sys

import numpy as np

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
SRC = os.path.join(REF, "tests", "numerics", "test_q4kwriter.py")
NEEDED_FUNCS = {"nearest_int", "nearest_int_away", "make_qkx2_quants", "get_scale_min_k4", "_f16_bits",
                "_f16_to_f32", "quantize_row_q4_K_ref", "_fixtures"}
NEEDED_CONSTS = {"F", "QK_K", "BLOCK_BYTES"}


def load():
    tree = ast.parse(open(SRC).read(), SRC)
    keep = []
    for node in tree.body:
        if isinstance(node, ast.FunctionDef) and node.name in NEEDED_FUNCS:
            keep.append(node)
        elif isinstance(node, ast.Assign) and all(isinstance(t, ast.Name) and t.id in NEEDED_CONSTS
                                                  for t in node.targets):
            keep.append(node)
    found = {n.name for n in keep if isinstance(n, ast.FunctionDef)}
    assert found == NEEDED_FUNCS, NEEDED_FUNCS - found
    ns = {"np": np, "struct": struct, "math": math}
    exec(compile(ast.Module(body=keep, type_ignores=[]), SRC, "exec"), ns)
    return ns


def main():
    ns = load()
    cases = []
    for name, x in ns["_fixtures"]().items():
        x = np.ascontiguousarray(x, dtype=np.float32)
        blob = ns["quantize_row_q4_K_ref"](x)
        cases.append({"name": name, "shape": list(x.shape), "input_f32": x.tobytes().hex(), "blob": bytes(blob).hex()})
    doc = {
        "what": "Q4_K writer vectors: quantize_row_q4_K_ref (llama.cpp ggml-quants.c at 3de52ac3) on the fixtures "
                "of the reference's tests/numerics/test_q4kwriter.py",
        "generator": "tests/golden/make_q4_k_writer_vectors.py",
        "cases": cases,
    }
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q4_k_writer.json")
    with open(out, "w") as fh:
        json.dump(doc, fh, indent=1)
    print(f"wrote {len(cases)} cases to {out}")


if __name__ == "__main__":
    main()
