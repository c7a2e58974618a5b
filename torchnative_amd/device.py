"""The `hip` member of the device namespace.

Mirrors torchnative/python/torchnative/device/__init__.py: the availability
record (`Availability`, :118-165) with its rules (an available device carries
no reason; an unavailable one carries a *name*, never prose alone; `kind`
says whether the answer was measured or declared), the eager device with
`available` / `require()` / `report()` (:307-361), the CUDA member that
passes its probe's reason through unchanged (:479-503), and `members()` /
`report()` (:789-803). The answer comes from `tn_probe` (include/tnhip.h),
which runs the HIP runtime, so it is always "measured".

Reasons:
  not_built   libtnhip.so has not been built (there is no host fallback);
  no_driver   the HIP runtime cannot enumerate devices;
  no_device   the runtime sees no GPU;
  wrong_arch  the current GPU is not a gfx950 (the library is built for it only).
"""

from __future__ import annotations

import re

from . import _lib

__all__ = ["Availability", "DeviceUnavailable", "HipDevice", "hip", "members", "report"]

REASONS = ("not_built", "no_driver", "no_device", "wrong_arch")


class DeviceUnavailable(RuntimeError):
    """This device is not usable in this process; the message names why."""


class Availability:
    """One availability answer and what produced it."""

    __slots__ = ("device", "available", "reason", "source", "kind", "detail")

    def __init__(self, device, available, source, kind, reason=None, detail=None):
        if kind not in ("measured", "declared"):
            raise ValueError(f"kind must be 'measured' or 'declared', got {kind!r}")
        if available and reason is not None:
            raise ValueError("an available device must not carry a refusal reason")
        if not available and not reason:
            raise ValueError(f"{device}: unavailable without a named reason")
        self.device, self.available, self.reason = device, bool(available), reason
        self.source, self.kind, self.detail = source, kind, dict(detail or {})

    def as_dict(self):
        return {"device": self.device, "available": self.available, "reason": self.reason, "source": self.source,
                "kind": self.kind, "detail": self.detail}

    def __repr__(self):
        state = "available" if self.available else f"unavailable ({self.reason})"
        return f"<Availability {self.device}: {state} via {self.source} [{self.kind}]>"


class HipDevice:
    """The MI355X (gfx950) behind libtnhip: an eager tensor destination."""

    __slots__ = ()
    type = "hip"
    eager = True
    source = "tn_probe (libtnhip)"

    def availability(self) -> Availability:
        try:
            L = _lib.lib()
        except _lib.HipLibraryMissing as e:
            return Availability("hip", False, self.source, "measured", reason="not_built", detail={"error": str(e)})
        from ._C import _hip_probe

        try:
            probe = _hip_probe()
        except NotImplementedError as e:
            msg = str(e)
            m = re.search(r"tnhip: (\w+):", msg)
            reason = m.group(1) if m and m.group(1) in REASONS else "unclassified"
            return Availability("hip", False, self.source, "measured", reason=reason, detail={"error": msg})
        del L
        return Availability("hip", True, self.source, "measured", detail=probe)

    @property
    def available(self) -> bool:
        return self.availability().available

    def require(self) -> "HipDevice":
        """Return self, or raise DeviceUnavailable naming the reason."""
        a = self.availability()
        if not a.available:
            raise DeviceUnavailable(f"torchnative_amd.device.hip is not available in this process -- reason: "
                                    f"{a.reason} (probe: {a.source})")
        return self

    def report(self) -> dict:
        return {"type": self.type, "eager": self.eager, **self.availability().as_dict()}

    # what the reference's `_cuda_counters` / `_vulkan_ops` expose for residency tests
    def counters(self) -> dict:
        from ._C import _hip_counters

        return _hip_counters()

    def ops(self) -> list:
        from ._C import _hip_ops

        return _hip_ops()

    def synchronize(self) -> None:
        from .tensor import synchronize

        synchronize()

    def __repr__(self):
        return "torchnative_amd.device.hip (eager)"


hip = HipDevice()


def members():
    """Every device this package provides, in a stable order."""
    return (hip,)


def report() -> dict:
    return {d.type: d.report() for d in members()}
