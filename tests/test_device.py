"""The hip device's availability: measured by running tn_probe, a negative
answer carries one of the reason codes, `ensure()` raises with that code, a
missing library reads as `not_built` (never a fallback), and on the GPU the
device is usable with the probe's properties and its counters move with the
work -- the checks the reference's tests/devices/cuda/test_cuda.py makes of
its CUDA member."""

import numpy as np
import pytest

from torchnative_amd import _lib
from torchnative_amd import device as D


def test_a_probe_result_carries_a_reason_exactly_when_unusable():
    with pytest.raises(ValueError, match="exactly one"):
        D.ProbeResult(True, "no_driver")
    with pytest.raises(ValueError, match="exactly one"):
        D.ProbeResult(False)
    with pytest.raises(ValueError, match="unknown reason code"):
        D.ProbeResult(False, "tired")
    assert D.ProbeResult(False, "no_device", {"error": "x"}).props == {"error": "x"}


def test_the_answer_comes_from_the_probe_and_names_its_reason():
    r = D.probe()
    st = D.hip.status()
    assert st["usable"] == r.usable and st["eager"] is True and set(D.report()) == {"hip"}
    if not r.usable:
        assert r.reason in D.REASONS
        with pytest.raises(D.DeviceUnavailable) as e:
            D.hip.ensure()
        assert e.value.reason == r.reason and r.reason in str(e.value)
        assert not D.hip.is_available()


def test_a_missing_library_is_not_built_not_a_fallback(monkeypatch):
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libtnhip.so")
    monkeypatch.setattr(_lib, "_lib", None)
    r = D.probe()
    assert not r.usable and r.reason == "not_built" and "no host fallback" in r.props["error"]


@pytest.mark.gpu
def test_on_the_gpu_the_device_is_usable_and_counts_its_work():
    import torchnative_amd as tn

    r = D.hip.ensure()
    assert r.usable and r.reason is None and r.props["arch"].startswith("gfx950") and D.hip.is_available()
    assert "torch._C._quantized_linear(q4_k)" in ",".join(D.hip.ops())
    tn._C._hip_counters_reset()
    before = D.hip.counters()
    x = tn.tensor(np.ones((1, 64), np.float32), device="hip")
    q = tn._quantize(tn.tensor(np.ones((8, 64), np.float32), device="hip"), "q8_0")
    tn._quantized_linear(x, q)
    D.hip.synchronize()
    after = D.hip.counters()
    assert after["dispatches"] >= before["dispatches"] + 2 and after["bytes_uploaded"] > before["bytes_uploaded"]
