"""The f32 prefill's stream-K partition (torchnative_amd/csrc/skgeo.h), the
same header the kernel compiles, built for the host with g++ and walked the
way k_fa_f32 walks it (tests/skgeo_check.cpp): every unit covered once by a
non-empty range, whole blocks written once, cut blocks' partials in distinct
slots that the merge's arithmetic finds again in workgroup order. Shapes
cover batch*heads 1-64, query and key lengths from 1 to 4096, causal and not,
both key tile sizes and grids of 1 to 1024 workgroups.
"""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "torchnative_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
def test_stream_k_partition(tmp_path):
    exe = tmp_path / "skgeo_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", CSRC, "-o", str(exe), os.path.join(HERE, "skgeo_check.cpp")],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok "), r.stdout
    assert int(r.stdout.split()[1]) > 8000
