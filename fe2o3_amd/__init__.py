"""fe2o3_amd -- MI355X (gfx950) implementation of fe2o3's dense-compute path.

The compute lives in libfe2o3_mi355x.so (hand-written HIP for gfx950 behind
the C-ABI of include/fe2o3_mi355x.h).  This package is the host side:
``runtime`` (context, streams, events, device buffers) and ``kernels`` (the
typed ``<kernel>_gpu.Kernel.load/prepare/launch`` surface).  There is no CPU
fallback: without the built library every call raises.
"""
from . import _lib  # noqa: F401

__all__ = ["runtime", "kernels"]
