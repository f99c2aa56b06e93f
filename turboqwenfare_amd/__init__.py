"""turboqwenfare_amd -- the MI355X (gfx950) HIP backend for TurboQwenFare's
MTP speculative-verify hot path: a Q4_0 group-quantised MoE expert FFN over
the k+1 verify rows and the acceptance sampling over vocab logits.

The compute lives in ``libtqf_hip.so`` (C ABI, ``include/tqf_hip.h``);
``backend.HipBackend`` is the host-side mirror of the reference's backend
seams, ``mtp`` the verify accounting and ``synth`` the seeded synthetic
workloads.
"""
from . import mtp, synth  # noqa: F401

__all__ = ["mtp", "synth", "backend", "build"]
