"""Is the hip device usable in this process, and if not, why not.

The answer comes from running the library's own probe (`tn_probe`,
include/tnhip.h), which asks the HIP runtime for the current device and
checks that it is a gfx950; nothing is inferred from the environment. A
negative answer always carries one of four reason codes, so callers and
tests can branch on the code rather than parse prose:

  not_built   libtnhip.so has not been built (there is no host fallback);
  no_driver   the HIP runtime cannot enumerate devices;
  no_device   the runtime sees no GPU;
  wrong_arch  the current GPU is not a gfx950 (the library is built for it only).

The reference's device namespace (torchnative/python/torchnative/device)
would take this as one more member: a small class registered there that
forwards its availability question to `probe()`.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field

from . import _lib

__all__ = ["ProbeResult", "DeviceUnavailable", "probe", "hip", "report", "REASONS"]

REASONS = ("not_built", "no_driver", "no_device", "wrong_arch")


class DeviceUnavailable(RuntimeError):
    """The hip device cannot be used here; `.reason` holds the code."""

    def __init__(self, reason: str, message: str):
        super().__init__(message)
        self.reason = reason


@dataclass(frozen=True)
class ProbeResult:
    """One run of the probe. `props` holds what tn_probe reported about the
    device (name, arch, CUs, HBM bytes, clock, device count) when usable,
    or the error text under "error" when not."""

    usable: bool
    reason: str | None = None
    props: dict = field(default_factory=dict)

    def __post_init__(self):
        if self.usable == (self.reason is not None):
            raise ValueError("a usable probe has no reason code and an unusable one has exactly one")
        if self.reason is not None and self.reason not in REASONS + ("unclassified",):
            raise ValueError(f"unknown reason code {self.reason!r}")


def probe() -> ProbeResult:
    """Run tn_probe now and classify the outcome."""
    try:
        _lib.lib()
    except _lib.HipLibraryMissing as e:
        return ProbeResult(False, "not_built", {"error": str(e)})
    from ._C import _hip_probe

    try:
        return ProbeResult(True, None, _hip_probe())
    except NotImplementedError as e:
        text = str(e)
        code = re.match(r"tnhip: (\w+):", text)
        reason = code.group(1) if code and code.group(1) in REASONS else "unclassified"
        return ProbeResult(False, reason, {"error": text})


class _Hip:
    """`torchnative_amd.device.hip`: the MI355X behind libtnhip, an eager
    device (every op runs when called; nothing is traced)."""

    name = "hip"

    def is_available(self) -> bool:
        return probe().usable

    def ensure(self) -> ProbeResult:
        """The probe result if the device is usable, else DeviceUnavailable
        carrying the reason code."""
        r = probe()
        if not r.usable:
            raise DeviceUnavailable(r.reason, f"hip device unusable ({r.reason}): {r.props.get('error', '')}")
        return r

    def status(self) -> dict:
        r = probe()
        return {"device": self.name, "usable": r.usable, "reason": r.reason, "eager": True, **r.props}

    def counters(self) -> dict:
        """Launches, uploads, host readbacks, refusals and workspace bytes
        since the last reset (tn_counters)."""
        from ._C import _hip_counters

        return _hip_counters()

    def ops(self) -> list:
        """The op names this backend executes (tn_ops); anything else is refused."""
        from ._C import _hip_ops

        return _hip_ops()

    def synchronize(self) -> None:
        from .tensor import synchronize

        synchronize()

    def __repr__(self):
        return "<torchnative_amd.device.hip>"


hip = _Hip()


def report() -> dict:
    """The status of every device this package provides, by name."""
    return {hip.name: hip.status()}
