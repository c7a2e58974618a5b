"""The `hip` device member (torchnative/python/torchnative/device/__init__.py
:118-165, :307-361, :479-503): availability is measured by tn_probe, an
unavailable device carries a named reason, `require()` raises naming it, and
on the GPU the member is available with the probe's detail and its counters
move with the work -- the checks tests/devices/cuda/test_cuda.py makes of the
CUDA member."""

import numpy as np
import pytest

from torchnative_amd import _lib
from torchnative_amd import device as D


def test_availability_records_follow_the_rules():
    with pytest.raises(ValueError, match="kind"):
        D.Availability("hip", True, "x", "guessed")
    with pytest.raises(ValueError, match="must not carry"):
        D.Availability("hip", True, "x", "measured", reason="no_driver")
    with pytest.raises(ValueError, match="without a named reason"):
        D.Availability("hip", False, "x", "measured")
    a = D.Availability("hip", False, "x", "declared", reason="not_built", detail={"k": 1})
    assert a.as_dict() == {"device": "hip", "available": False, "reason": "not_built", "source": "x",
                           "kind": "declared", "detail": {"k": 1}}


def test_the_answer_is_measured_and_names_its_reason():
    a = D.hip.availability()
    assert a.kind == "measured" and a.source.startswith("tn_probe")
    if not a.available:
        assert a.reason in D.REASONS
        with pytest.raises(D.DeviceUnavailable, match=f"reason: {a.reason}"):
            D.hip.require()
    rep = D.report()
    assert set(rep) == {"hip"} and rep["hip"]["eager"] is True and D.members() == (D.hip,)


def test_a_missing_library_is_not_built_not_a_fallback(monkeypatch):
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libtnhip.so")
    monkeypatch.setattr(_lib, "_lib", None)
    a = D.hip.availability()
    assert not a.available and a.reason == "not_built" and "no host fallback" in a.detail["error"]


@pytest.mark.gpu
def test_on_the_gpu_the_member_is_available_and_counts_its_work():
    import torchnative_amd as tn

    a = D.hip.require().availability()
    assert a.available and a.reason is None and a.detail["arch"].startswith("gfx950")
    assert "torch._C._quantized_linear(q4_k)" in ",".join(D.hip.ops())
    tn._C._hip_counters_reset()
    before = D.hip.counters()
    x = tn.tensor(np.ones((1, 64), np.float32), device="hip")
    q = tn._quantize(tn.tensor(np.ones((8, 64), np.float32), device="hip"), "q8_0")
    tn._quantized_linear(x, q)
    D.hip.synchronize()
    after = D.hip.counters()
    assert after["dispatches"] >= before["dispatches"] + 2 and after["bytes_uploaded"] > before["bytes_uploaded"]
