"""Host runtime over the C-ABI: context, streams, events and device buffers.

Mirrors the shape of fe2o3-core's HIP-backed runtime (``GpuContext``,
``Stream``, ``Event``, ``DeviceBuffer``; crates/fe2o3-core/src/lib.rs:18-53,
context.rs:11-62, stream.rs:44-80, memory.rs:91-140): the context binds the
device before every operation (context.rs:52-54), buffers are owned by the
caller and freed on drop, and every failing call raises ``Fe2o3Error``
carrying the status.
"""
from __future__ import annotations

import ctypes as C
import threading

import numpy as np

from . import _lib
from ._lib import Fe2o3HipDeviceProperties

H2D, D2H, D2D = 1, 2, 3


class Fe2o3Error(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = int(status)
        super().__init__(f"{what}: status {status} ({_lib.status_string(status)})")


def check(status: int, what: str) -> None:
    if status != 0:
        raise Fe2o3Error(status, what)


class Stream:
    """A HIP stream at the default priority (crates/fe2o3-core/src/stream.rs)."""

    def __init__(self, ctx: "GpuContext"):
        self.ctx = ctx
        h = C.c_void_p()
        ctx.bind()
        check(_lib.lib().fe2o3_rt_stream_create(C.byref(h)), "stream create")
        self.handle = h.value

    def synchronize(self) -> None:
        check(_lib.lib().fe2o3_rt_stream_synchronize(self.handle), "stream synchronize")

    def close(self) -> None:
        if self.handle is not None:
            _lib.lib().fe2o3_rt_stream_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self, ctx: "GpuContext", timing: bool = True):
        h = C.c_void_p()
        ctx.bind()
        check(_lib.lib().fe2o3_rt_event_create(C.byref(h), 0 if timing else 2), "event create")
        self.handle = h.value

    def record(self, stream: Stream | None) -> None:
        check(_lib.lib().fe2o3_rt_event_record(self.handle, stream_handle(stream)), "event record")

    def synchronize(self) -> None:
        check(_lib.lib().fe2o3_rt_event_synchronize(self.handle), "event synchronize")

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float()
        check(_lib.lib().fe2o3_rt_event_elapsed_ms(C.byref(ms), self.handle, later.handle),
              "event elapsed")
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle is not None:
                _lib.lib().fe2o3_rt_event_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


def stream_handle(stream) -> int | None:
    if stream is None:
        return None
    return stream.handle


class DeviceBuffer:
    """Caller-owned device allocation of ``count`` elements of ``dtype``."""

    def __init__(self, ctx: "GpuContext", count: int, dtype):
        self.ctx = ctx
        self.dtype = np.dtype(dtype)
        self.count = int(count)
        self.nbytes = self.count * self.dtype.itemsize
        p = C.c_void_p()
        ctx.bind()
        check(_lib.lib().fe2o3_rt_malloc(C.byref(p), max(self.nbytes, 1)), "malloc")
        self.ptr = p.value

    @property
    def len(self) -> int:
        return self.count

    def upload(self, host: np.ndarray, stream: Stream | None = None) -> "DeviceBuffer":
        host = np.ascontiguousarray(host, dtype=self.dtype).ravel()
        if host.size != self.count:
            raise ValueError(f"upload of {host.size} elements into a buffer of {self.count}")
        if self.nbytes:
            check(_lib.lib().fe2o3_rt_memcpy(self.ptr, host.ctypes.data, self.nbytes, H2D),
                  "memcpy H2D")
        return self

    def download(self) -> np.ndarray:
        out = np.empty(self.count, self.dtype)
        if self.nbytes:
            check(_lib.lib().fe2o3_rt_memcpy(out.ctypes.data, self.ptr, self.nbytes, D2H),
                  "memcpy D2H")
        return out

    def view(self, offset: int, count: int) -> "DeviceBuffer":
        """Non-owning window of ``count`` elements starting at element
        ``offset`` (used for guard-banded test allocations)."""
        if offset < 0 or count < 0 or offset + count > self.count:
            raise ValueError("view out of range")
        v = DeviceBuffer.__new__(_View)
        v.ctx, v.dtype, v.count = self.ctx, self.dtype, int(count)
        v.nbytes = v.count * self.dtype.itemsize
        v.ptr = self.ptr + offset * self.dtype.itemsize
        v.owner = self
        return v

    def fill_bytes(self, value: int, stream: Stream | None = None) -> None:
        check(_lib.lib().fe2o3_rt_memset_async(self.ptr, value, self.nbytes,
                                               stream_handle(stream)), "memset")

    def free(self) -> None:
        if getattr(self, "ptr", None):
            _lib.lib().fe2o3_rt_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class _View(DeviceBuffer):
    def free(self) -> None:  # the owner frees
        self.ptr = None


class GpuContext:
    """Device binding plus the 312-byte property record
    (crates/fe2o3-core/src/context.rs:11-62)."""

    _current = None
    _lock = threading.Lock()

    def __init__(self, device: int = 0):
        L = _lib.lib()
        check(L.fe2o3_rt_init(0), "hipInit")
        n = C.c_int32()
        check(L.fe2o3_rt_get_device_count(C.byref(n)), "device count")
        if n.value <= device:
            raise Fe2o3Error(100, f"device {device} not present ({n.value} visible)")
        self.device = device
        self.bind()
        check(L.fe2o3_rt_require_gfx950(device), "gfx950 required")
        self.props = Fe2o3HipDeviceProperties()
        check(L.fe2o3HipGetDeviceProperties(device, C.byref(self.props)), "device properties")
        cu, clk, mclk, bus = C.c_int32(), C.c_int32(), C.c_int32(), C.c_int32()
        check(L.fe2o3_rt_device_rates(device, C.byref(cu), C.byref(clk), C.byref(mclk),
                                      C.byref(bus)), "device rates")
        self.compute_units = cu.value
        self.clock_khz = clk.value
        self.memory_clock_khz = mclk.value
        self.memory_bus_bits = bus.value

    @classmethod
    def current(cls, device: int = 0) -> "GpuContext":
        with cls._lock:
            if cls._current is None or cls._current.device != device:
                cls._current = GpuContext(device)
            return cls._current

    @property
    def arch(self) -> str:
        return self.props.gcn_arch_name.decode()

    def bind(self) -> None:
        check(_lib.lib().fe2o3_rt_set_device(self.device), "set device")

    def synchronize(self) -> None:
        check(_lib.lib().fe2o3_rt_device_synchronize(), "device synchronize")

    def stream(self) -> Stream:
        return Stream(self)

    def alloc(self, count: int, dtype) -> DeviceBuffer:
        return DeviceBuffer(self, count, dtype)

    def to_device(self, host: np.ndarray, dtype=None) -> DeviceBuffer:
        host = np.asarray(host)
        buf = DeviceBuffer(self, host.size, dtype or host.dtype)
        return buf.upload(host)
