"""Host side of the typed launch surface (fe2o3_amd/kernels.py), no GPU: a
prepared launch holds the slices it was given, so a buffer passed as a
temporary (``prepare(ctx.to_device(x), ...)``) is not collected, and its
device memory not freed, before the launch runs.  Mirrors the borrow the
reference's typed launch holds on its slices
(crates/fe2o3-host/src/loaded_kernel.rs:420-432)."""
from __future__ import annotations

import gc
import weakref

import numpy as np


class _FakeBuffer:
    """A DeviceBuffer that owns no device memory (no GPU here); records
    whether it was freed."""

    freed = 0

    @classmethod
    def make(cls, count, dtype):
        from fe2o3_amd.runtime import DeviceBuffer

        class Fake(DeviceBuffer):
            def free(self):
                if getattr(self, "ptr", None):
                    _FakeBuffer.freed += 1
                    self.ptr = None

        b = Fake.__new__(Fake)
        b.ctx, b.dtype, b.count = None, np.dtype(dtype), int(count)
        b.nbytes = b.count * b.dtype.itemsize
        b.ptr = 0x1000
        return b


def test_prepared_launch_keeps_temporary_slices_alive():
    from fe2o3_amd import kernels
    kern = kernels.tiled_gemm_general_v1_gpu.Kernel(ctx=None)
    _FakeBuffer.freed = 0
    prepared = kern.prepare(_FakeBuffer.make(6, np.uint16), _FakeBuffer.make(6, np.uint16),
                            _FakeBuffer.make(4, np.float32), 2, 2, 3, 3, 2, 2, 1.0, 0.0)
    refs = [weakref.ref(b) for b in prepared.buffers]
    gc.collect()
    assert _FakeBuffer.freed == 0
    assert all(r() is not None for r in refs)
    assert prepared.args[0] == 0x1000 and prepared.args[1] == 6
    del prepared
    gc.collect()
    assert _FakeBuffer.freed == 3
    assert all(r() is None for r in refs)
