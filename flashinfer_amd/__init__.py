"""MI355X-native fused MoE (FP8 block-scaled, DeepSeek routing) for gfx950.

``flashinfer_amd.kernel.run`` is the drop-in for the reference's
``kernel.py::run``; the compute lives in ``libmi_moe.so`` (HIP, gfx950).
"""
from .kernel import run, route  # noqa: F401

__all__ = ["run", "route"]
