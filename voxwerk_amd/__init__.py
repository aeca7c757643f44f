"""voxwerk_amd — voxwerk's per-step token sampler as a gfx950 (MI355X) HIP library.

The product is ``lib/libvxs.so`` (C ABI in ``include/vxs_sampler.h``); this package holds its HIP
sources (``csrc/``), the Python mirror of the reference's sampling surface (``sampler``), the
deterministic synthetic workloads (``workloads``) and the build recipe (``build``).
"""
from . import _lib  # noqa: F401

__all__ = ["sampler", "generate", "workloads", "build"]
__version__ = "0.1.0"
