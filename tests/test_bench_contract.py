"""bench.py's contract pieces that need no GPU: the measured HBM traffic each
config's roofline object carries comes from a committed rocprofv3 summary,
and `--gpus` above one is refused with a message instead of running."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


@pytest.mark.parametrize("name,lo,hi", [
    ("flash_bf16_c2_traffic.md", 6_365_184, 40e6),     # C2: at least its algorithmic bytes
    ("q4_gemv_c1.md", 515_901_696, 600e6),             # C1, 1,024 weight copies
    ("flash_f32_c2.md", 12_656_640, 200e6),            # C2 in f32, partials included
    ("q4_gemm_c3.md", 51_904_512, 200e6),              # C3
    ("decode_attention_c4.md", 179_662_848, 200e6),    # C4
])
def test_each_profile_carries_its_traffic(name, lo, hi):
    t = bench.profiled_traffic(name)
    assert t is not None, name
    assert lo <= t <= hi, (name, t)


def test_a_missing_profile_gives_none():
    assert bench.profiled_traffic("no_such_profile.md") is None


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr) or "1 GPU" in (r.stdout + r.stderr), r.stdout + r.stderr
