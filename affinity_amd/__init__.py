"""affinity_amd: MI355X (gfx950) routed-expert hot path for affinity's 2.875-bpw experts.

The compute lives in libaffx.so (HIP, C-ABI in include/affx.h); this package is the host-side
mirror of the reference's expert interface (affinity_amd.experts) and the build step
(affinity_amd.build). Importing it does not touch the GPU.
"""
from ._lib import AffxDeclined, AffxError, lib  # noqa: F401

__all__ = ["AffxDeclined", "AffxError", "lib"]
