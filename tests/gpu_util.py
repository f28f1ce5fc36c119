"""Helpers for the GPU parity tests: guard-banded device buffers (the
reference's hardware harnesses surround every allocation with canaries and
check inputs are unchanged, e.g.
examples/tiled_gemm_general_v1/hardware-harness/src/lib.rs:69-77,1629-1638)
and the BASELINE relative-error metric."""
from __future__ import annotations

import numpy as np

GUARD = 64  # elements on each side


def guard_pattern(dtype, n):
    dtype = np.dtype(dtype)
    if dtype == np.float32:
        return np.full(n, 0x7FC0DEAD, np.uint32).view(np.float32)  # NaN payload canary
    if dtype == np.uint16:
        return np.full(n, 0x7FDE, np.uint16)
    if dtype == np.uint32:
        return np.full(n, 0xDEADBEEF, np.uint32)
    if dtype == np.int32:
        return np.full(n, 0xDEADBEEF, np.uint32).view(np.int32)
    if dtype == np.uint8:
        return np.full(n, 0xA5, np.uint8)
    raise TypeError(dtype)


class Guarded:
    """A device allocation of GUARD + n + GUARD elements; ``body`` is the
    n-element window handed to the kernel."""

    def __init__(self, ctx, host_body, dtype=None):
        host_body = np.ascontiguousarray(host_body, dtype=dtype).ravel()
        self.dtype = host_body.dtype
        self.n = host_body.size
        g = guard_pattern(self.dtype, GUARD)
        self.initial = np.concatenate([g, host_body, g])
        self.full = ctx.to_device(self.initial)
        self.body = self.full.view(GUARD, self.n)

    def download(self):
        return self.full.download()[GUARD:GUARD + self.n]

    def guards_intact(self) -> bool:
        f = self.full.download()
        g = guard_pattern(self.dtype, GUARD)
        return (f[:GUARD].tobytes() == g.tobytes()) and (f[GUARD + self.n:].tobytes() == g.tobytes())

    def unchanged(self) -> bool:
        return self.full.download().tobytes() == self.initial.tobytes()


def rel_err(got, ref) -> float:
    """max |y - yhat| / max |yhat| (the BASELINE relative-error metric)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = np.max(np.abs(ref))
    if denom == 0:
        return float(np.max(np.abs(got - ref)))
    return float(np.max(np.abs(got - ref)) / denom)


def bf16_to_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_same(got, ref, what=""):
    """Bitwise equality of two arrays with a short report (never a full
    element diff, which is slow for large arrays)."""
    g = np.ascontiguousarray(got)
    r = np.ascontiguousarray(ref)
    assert g.shape == r.shape, (what, g.shape, r.shape)
    gb = g.view(np.uint8).reshape(g.size, -1) if g.size else g
    rb = r.view(np.uint8).reshape(r.size, -1) if r.size else r
    bad = np.nonzero(np.any(gb != rb, axis=1))[0] if g.size else np.array([], int)
    if bad.size:
        i = int(bad[0])
        raise AssertionError(f"{what}: {bad.size} of {g.size} elements differ; first at {i}: "
                             f"got {g.ravel()[i]!r} want {r.ravel()[i]!r}")
