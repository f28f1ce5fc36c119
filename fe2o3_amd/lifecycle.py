"""Typed, linear host mirror of the exact LDS GEMM lifecycle
(crates/fe2o3-host/src/generated_lds_gemm_lifecycle.rs) over the C-ABI
fe2o3_lds_gemm_slice1_* entry points.

    joined = join_exact_lds_gemm_slice1_v1(a, b, c)          # :276
    loaded = joined.load()                                    # :298 (HIP adapter)
    completed = loaded.dispatch_and_wait()                    # :391
    receipt = completed.unload()                              # :522

Each step consumes its value: a spent value raises StateError, as a moved
Rust value cannot be used.  A value dropped while it still owns the handle
releases it, which unloads a loaded executable (the reference's Drop).
Errors carry the reference's error kind and drifted field.

`load(adapter)` accepts a RuntimeAdapter: a Python object whose methods
implement the callback table (used by the CPU tests to observe and
fault-inject the lifecycle without a GPU).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from . import _lib
from .runtime import Fe2o3Error

JOINED, LOADED, COMPLETED, FAILED = 1, 2, 3, 4
ERR_JOIN, ERR_LOAD, ERR_DISPATCH, ERR_STATE = -27, -28, -29, -30

KINDS = {
    0: "None", 1: "ImportIdentity", 2: "ProfileIdentity", 3: "Contract", 4: "FinalizedOutput",
    5: "ContractField", 6: "BufferContract", 7: "HostLengthIdentity", 8: "HostField",
    9: "Length", 10: "NullAddress", 11: "Alignment", 12: "OutputOverlap",
    13: "RegionAddressOverflow",
    20: "ContextIdentity", 21: "EnvironmentAdapter", 22: "Environment", 23: "LoadAdapter",
    24: "LoadObservation", 25: "KernelAdapter", 26: "KernelObservation",
    27: "ResourceAdapter", 28: "ResourceObservation",
    40: "ImplicitAdapter", 41: "ImplicitObservation", 42: "ExplicitKernargMutation",
    43: "DispatchAdapter", 44: "DispatchObservation", 14: "ReceiptField",
}


class Slice1Error(Fe2o3Error):
    """A refused lifecycle step: `kind` names the reference's error variant,
    `field` the drifted field, `index` the buffer where one is named."""

    def __init__(self, status: int, err: _lib.Fe2o3Slice1ErrorV1 | None, what: str):
        super().__init__(status, what)
        err = err or _lib.Fe2o3Slice1ErrorV1()
        self.kind = KINDS.get(err.kind, str(err.kind))
        self.field = err.field.decode()
        self.index = err.index
        self.adapter_status = err.adapter_status
        self.expected, self.actual = err.expected, err.actual

    def __str__(self):
        detail = self.kind + (f"({self.field})" if self.field else "")
        if self.index >= 0:
            detail += f"[{self.index}]"
        return f"{super().__str__()}: {detail}"


class JoinError(Slice1Error):
    pass


class LoadError(Slice1Error):
    pass


class DispatchError(Slice1Error):
    pass


class StateError(Slice1Error):
    pass


def _raise(status: int, err, what: str):
    cls = {ERR_JOIN: JoinError, ERR_LOAD: LoadError, ERR_DISPATCH: DispatchError,
           ERR_STATE: StateError}.get(status, Slice1Error)
    raise cls(status, err, what)


def artifact() -> _lib.Fe2o3Slice1ArtifactV1:
    out = _lib.Fe2o3Slice1ArtifactV1()
    _check(_lib.lib().fe2o3_lds_gemm_slice1_artifact_v1(C.byref(out)), "artifact")
    return out


def join_facts() -> _lib.Fe2o3Slice1JoinFactsV1:
    out = _lib.Fe2o3Slice1JoinFactsV1()
    _check(_lib.lib().fe2o3_lds_gemm_slice1_join_facts_v1(C.byref(out)), "join facts")
    return out


def validate_join(facts: _lib.Fe2o3Slice1JoinFactsV1) -> None:
    err = _lib.Fe2o3Slice1ErrorV1()
    rc = _lib.lib().fe2o3_lds_gemm_slice1_validate_join_v1(C.byref(facts), C.byref(err))
    if rc:
        _raise(rc, err, "validate_join")


def sha256(data: bytes) -> bytes:
    out = (C.c_uint8 * 32)()
    _check(_lib.lib().fe2o3_sha256_v1(data, len(data), C.byref(out)), "sha256")
    return bytes(out)


def context_identity(device: int) -> bytes:
    out = (C.c_uint8 * 16)()
    _check(_lib.lib().fe2o3_lds_gemm_slice1_context_identity_v1(device, C.byref(out)),
           "context identity")
    return bytes(out)


def _check(rc: int, what: str) -> None:
    if rc:
        raise Fe2o3Error(rc, what)


def _region(x, dtype_size: int):
    """(address, element count) of a DeviceBuffer, a numpy array or a pair."""
    if isinstance(x, tuple):
        return int(x[0] or 0), int(x[1])
    if hasattr(x, "ptr") and hasattr(x, "count"):
        return int(x.ptr or 0), int(x.count)
    if hasattr(x, "ctypes"):
        return int(x.ctypes.data), int(x.size)
    raise TypeError(f"cannot take a region of {type(x).__name__}")


class RuntimeAdapter:
    """Base class of a Python-implemented adapter.  Subclasses override the
    callbacks (same names and arguments as Fe2o3Slice1AdapterV1, minus
    `self`); each returns 0 on success.  table() builds the C table; the
    ctypes thunks stay alive as long as this object."""

    def context_identity(self, identity) -> int:
        return -1

    def observe_environment(self, out) -> int:
        return -1

    def load_executable(self, data, byte_len, digest, executable, out) -> int:
        return -1

    def resolve_kernel(self, executable, symbol, kernel, out) -> int:
        return -1

    def observe_resources(self, executable, kernel, out) -> int:
        return -1

    def initialize_implicit_kernarg(self, executable, kernel, geometry, explicit_bytes,
                                    implicit_offset, implicit_bytes, kernarg, kernarg_bytes,
                                    out) -> int:
        return -1

    def launch_and_wait(self, executable, kernel, geometry, kernarg, kernarg_bytes, out) -> int:
        return -1

    def drop_kernel(self, kernel) -> None:
        pass

    def unload_executable(self, executable, out) -> int:
        return -1

    def drop_adapter(self) -> None:
        pass

    def table(self) -> _lib.Fe2o3Slice1AdapterV1:
        if getattr(self, "_table", None) is None:
            L = _lib
            self._thunks = [
                L.SLICE1_CONTEXT_FN(lambda s, ident: self.context_identity(ident.contents)),
                L.SLICE1_ENVIRONMENT_FN(lambda s, out: self.observe_environment(out.contents)),
                L.SLICE1_LOAD_FN(lambda s, d, n, dg, exe, out: self.load_executable(
                    d, n, dg.contents, exe, out.contents)),
                L.SLICE1_RESOLVE_FN(lambda s, exe, sym, k, out: self.resolve_kernel(
                    exe, sym, k, out.contents)),
                L.SLICE1_RESOURCES_FN(lambda s, exe, k, out: self.observe_resources(
                    exe, k, out.contents)),
                L.SLICE1_IMPLICIT_FN(lambda s, exe, k, g, eb, io, ib, ka, kb, out:
                                     self.initialize_implicit_kernarg(
                                         exe, k, g.contents, eb, io, ib, ka, kb, out.contents)),
                L.SLICE1_LAUNCH_FN(lambda s, exe, k, g, ka, kb, out: self.launch_and_wait(
                    exe, k, g.contents, ka, kb, out.contents)),
                L.SLICE1_DROP_KERNEL_FN(lambda s, k: self.drop_kernel(k)),
                L.SLICE1_UNLOAD_FN(lambda s, exe, out: self.unload_executable(exe, out.contents)),
                L.SLICE1_DROP_ADAPTER_FN(lambda s: self.drop_adapter()),
            ]
            self._table = L.Fe2o3Slice1AdapterV1(None, *self._thunks)
        return self._table


class _Handle:
    """Owner of one C lifecycle handle and of everything its callbacks need
    kept alive (the lease-release thunk, a Python adapter).  `prefix` names
    the entry-point family that drives it."""

    def __init__(self, ptr: int, release_thunk, device: int,
                 prefix: str = "fe2o3_lds_gemm_slice1"):
        self.ptr = ptr
        self.release_thunk = release_thunk
        self.device = device
        self.adapter = None
        self.prefix = prefix

    def fn(self, name: str):
        return getattr(_lib.lib(), f"{self.prefix}_{name}")

    def observe(self) -> _lib.Fe2o3Slice1ObservationV1:
        out = _lib.Fe2o3Slice1ObservationV1()
        _check(self.fn("observe_v1")(self.ptr, C.byref(out)), "observe")
        return out

    def release(self) -> None:
        if self.ptr:
            ptr, self.ptr = self.ptr, None
            self.fn("release_v1")(ptr)


class _Linear:
    def __init__(self, handle: _Handle):
        self._handle = handle

    def _take(self) -> _Handle:
        h, self._handle = self._handle, None
        if h is None or not h.ptr:
            raise StateError(ERR_STATE, None, f"{type(self).__name__} was already consumed")
        return h

    def observation(self) -> _lib.Fe2o3Slice1ObservationV1:
        if self._handle is None:
            raise StateError(ERR_STATE, None, f"{type(self).__name__} was already consumed")
        return self._handle.observe()

    def release(self) -> None:
        """Drop: unloads first when an executable is held."""
        h, self._handle = self._handle, None
        if h is not None:
            h.release()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class JoinedExactLdsGemmSlice1V1(_Linear):
    def __init__(self, handle: _Handle):
        super().__init__(handle)
        a = artifact()
        self.finalizer_identity = bytes(a.finalizer_identity)
        self.import_identity = bytes(a.import_identity)
        self.profile_identity = bytes(a.profile_identity)

    def load(self, adapter: RuntimeAdapter | None = None) -> "LoadedExactLdsGemmSlice1V1":
        h = self._take()
        if adapter is None:
            table = _lib.Fe2o3Slice1AdapterV1()
            rc = _lib.lib().fe2o3_lds_gemm_slice1_hip_adapter_v1(h.device, C.byref(table))
            if rc:
                h.release()
                raise Fe2o3Error(rc, "HIP adapter")
        else:
            table = adapter.table()
            h.adapter = adapter
        err = _lib.Fe2o3Slice1ErrorV1()
        rc = _lib.lib().fe2o3_lds_gemm_slice1_load_v1(h.ptr, C.byref(table), C.byref(err))
        if rc:
            h.release()
            _raise(rc, err, "load")
        return LoadedExactLdsGemmSlice1V1(h)


class LoadedExactLdsGemmSlice1V1(_Linear):
    def dispatch_and_wait(self) -> "CompletedExactLdsGemmSlice1V1":
        h = self._take()
        err = _lib.Fe2o3Slice1ErrorV1()
        rc = _lib.lib().fe2o3_lds_gemm_slice1_dispatch_and_wait_v1(h.ptr, C.byref(err))
        if rc:
            h.release()
            _raise(rc, err, "dispatch_and_wait")
        return CompletedExactLdsGemmSlice1V1(h)


class CompletedExactLdsGemmSlice1V1(_Linear):
    def __init__(self, handle: _Handle):
        super().__init__(handle)
        o = handle.observe()
        self.executable_object = bytes(o.load.executable_object)
        self.kernel_object = bytes(o.resolution.kernel_object)
        self.dispatch_identity = bytes(o.dispatch_identity)

    def unload(self) -> "UnloadedExactLdsGemmSlice1V1":
        h = self._take()
        receipt = _lib.Fe2o3Slice1ReceiptV1()
        rc = _lib.lib().fe2o3_lds_gemm_slice1_unload_v1(h.ptr, C.byref(receipt))
        if rc:
            h.release()
            _raise(rc, None, "unload")
        h.ptr = None  # freed by the unload
        return UnloadedExactLdsGemmSlice1V1(
            bytes(receipt.finalizer_identity), bytes(receipt.import_identity),
            bytes(receipt.profile_identity), bytes(receipt.executable_object),
            bytes(receipt.kernel_object), bytes(receipt.dispatch_identity),
            bytes(receipt.unload_identity))


@dataclass(frozen=True)
class UnloadedExactLdsGemmSlice1V1:
    """Terminal, inert receipt (generated_lds_gemm_lifecycle.rs:569-607)."""

    finalizer_identity: bytes
    import_identity: bytes
    profile_identity: bytes
    executable_object: bytes
    kernel_object: bytes
    dispatch_identity: bytes
    unload_identity: bytes


def join_exact_lds_gemm_slice1_v1(a, b, c, device: int = 0,
                                  on_release=None) -> JoinedExactLdsGemmSlice1V1:
    """Prepares the host request for A, B (256 bf16 values each) and C (256
    f32) and joins it to the library's code object.  `on_release()` runs
    exactly once, when the lifecycle stops referring to A, B and C."""
    pa, na = _region(a, 2)
    pb, nb = _region(b, 2)
    pc, nc = _region(c, 4)
    thunk = _lib.SLICE1_RELEASE_FN(lambda user: on_release() if on_release else None)
    out = C.c_void_p()
    err = _lib.Fe2o3Slice1ErrorV1()
    rc = _lib.lib().fe2o3_lds_gemm_slice1_join_v1(pa or None, na, pb or None, nb, pc or None, nc,
                                                  device, thunk, None, C.byref(out),
                                                  C.byref(err))
    if rc:
        _raise(rc, err, "join")
    return JoinedExactLdsGemmSlice1V1(_Handle(out.value, thunk, device))


# ---- protected profile lifecycles -------------------------------------------------------
#
# crates/fe2o3-host/src/flash_attention_v1_lifecycle.rs,
# protected_row_softmax_v1_lifecycle.rs and moe_top2_v1_lifecycle.rs over
# the fe2o3_protected_* entry points: the same linear join -> load ->
# dispatch_and_wait -> unload, each profile over its own embedded code
# object.

FLASH_ATTENTION_V1, ROW_SOFTMAX_V1, MOE_TOP2_V1 = 1, 2, 3


def protected_profile(profile: int) -> _lib.Fe2o3ProtectedProfileV1:
    out = _lib.Fe2o3ProtectedProfileV1()
    _check(_lib.lib().fe2o3_protected_profile_v1(profile, C.byref(out)), "protected profile")
    return out


def protected_artifact(profile: int) -> _lib.Fe2o3ProtectedArtifactV1:
    out = _lib.Fe2o3ProtectedArtifactV1()
    _check(_lib.lib().fe2o3_protected_artifact_v1(profile, C.byref(out)), "protected artifact")
    return out


def protected_join_facts(profile: int) -> _lib.Fe2o3ProtectedJoinFactsV1:
    out = _lib.Fe2o3ProtectedJoinFactsV1()
    _check(_lib.lib().fe2o3_protected_join_facts_v1(profile, C.byref(out)), "join facts")
    return out


def protected_validate_join(facts: _lib.Fe2o3ProtectedJoinFactsV1) -> None:
    err = _lib.Fe2o3Slice1ErrorV1()
    rc = _lib.lib().fe2o3_protected_validate_join_v1(C.byref(facts), C.byref(err))
    if rc:
        _raise(rc, err, "validate_join")


class JoinedProtectedV1(_Linear):
    def __init__(self, handle: _Handle, profile: int):
        super().__init__(handle)
        self.profile = profile
        a = protected_artifact(profile)
        self.identity = bytes(a.identity)
        self.artifact_identity = bytes(a.artifact_identity)

    def load(self, adapter: RuntimeAdapter | None = None) -> "LoadedProtectedV1":
        h = self._take()
        if adapter is None:
            table = _lib.Fe2o3Slice1AdapterV1()
            rc = _lib.lib().fe2o3_lds_gemm_slice1_hip_adapter_v1(h.device, C.byref(table))
            if rc:
                h.release()
                raise Fe2o3Error(rc, "HIP adapter")
        else:
            table = adapter.table()
            h.adapter = adapter
        err = _lib.Fe2o3Slice1ErrorV1()
        rc = _lib.lib().fe2o3_protected_load_v1(h.ptr, C.byref(table), C.byref(err))
        if rc:
            h.release()
            _raise(rc, err, "load")
        return LoadedProtectedV1(h, self.profile)


class LoadedProtectedV1(_Linear):
    def __init__(self, handle: _Handle, profile: int):
        super().__init__(handle)
        self.profile = profile

    def dispatch_and_wait(self) -> "CompletedProtectedV1":
        h = self._take()
        err = _lib.Fe2o3Slice1ErrorV1()
        rc = _lib.lib().fe2o3_protected_dispatch_and_wait_v1(h.ptr, C.byref(err))
        if rc:
            h.release()
            _raise(rc, err, "dispatch_and_wait")
        return CompletedProtectedV1(h, self.profile)


class CompletedProtectedV1(_Linear):
    def __init__(self, handle: _Handle, profile: int):
        super().__init__(handle)
        self.profile = profile
        o = handle.observe()
        self.executable_object = bytes(o.load.executable_object)
        self.kernel_object = bytes(o.resolution.kernel_object)
        self.dispatch_identity = bytes(o.dispatch_identity)

    def unload(self) -> "UnloadedProtectedV1":
        h = self._take()
        receipt = _lib.Fe2o3ProtectedReceiptV1()
        rc = _lib.lib().fe2o3_protected_unload_v1(h.ptr, C.byref(receipt))
        if rc:
            h.release()
            _raise(rc, None, "unload")
        h.ptr = None  # freed by the unload
        return UnloadedProtectedV1(self.profile, bytes(receipt.identity),
                                   bytes(receipt.artifact_identity),
                                   bytes(receipt.executable_object), bytes(receipt.kernel_object),
                                   bytes(receipt.dispatch_identity),
                                   bytes(receipt.unload_identity))


@dataclass(frozen=True)
class UnloadedProtectedV1:
    """Terminal, inert receipt (e.g. UnloadedFlashAttentionV1,
    flash_attention_v1_lifecycle.rs:503-556)."""

    profile: int
    identity: bytes
    artifact_identity: bytes
    executable_object: bytes
    kernel_object: bytes
    dispatch_identity: bytes
    unload_identity: bytes


def join_protected_v1(profile: int, regions, device: int = 0,
                      on_release=None) -> JoinedProtectedV1:
    """Prepares the host request -- `regions` in the profile's role order,
    each a DeviceBuffer, a numpy array or an (address, elements) pair -- and
    joins it to the profile's code object.  `on_release()` runs exactly
    once, when the lifecycle stops referring to the regions."""
    arr = (_lib.Fe2o3ProtectedRegionV1 * max(1, len(regions)))()
    for i, r in enumerate(regions):
        addr, n = _region(r, 4)
        arr[i] = _lib.Fe2o3ProtectedRegionV1(addr or None, n)
    thunk = _lib.SLICE1_RELEASE_FN(lambda user: on_release() if on_release else None)
    out = C.c_void_p()
    err = _lib.Fe2o3Slice1ErrorV1()
    rc = _lib.lib().fe2o3_protected_join_v1(profile, arr, len(regions), device, thunk, None,
                                            C.byref(out), C.byref(err))
    if rc:
        _raise(rc, err, "join")
    return JoinedProtectedV1(_Handle(out.value, thunk, device, "fe2o3_protected"), profile)


def join_flash_attention_v1(q, k, v, output, device: int = 0, on_release=None):
    """flash_attention_v1_lifecycle.rs:228 join_flash_attention_v1: Q, K, V,
    output (128 f32 each)."""
    return join_protected_v1(FLASH_ATTENTION_V1, [q, k, v, output], device, on_release)


def join_row_softmax_v1(input, output, device: int = 0, on_release=None):
    """protected_row_softmax_v1_lifecycle.rs: input, output (64 f32 each)."""
    return join_protected_v1(ROW_SOFTMAX_V1, [input, output], device, on_release)


def join_moe_top2_v1(logits, top2_experts, requested_counts, admitted_counts, expert_offsets,
                     route_slots, permutation, inverse, device: int = 0, on_release=None):
    """moe_top2_v1_lifecycle.rs: logits (32 f32) and the seven u32 routing
    outputs (16, 4, 4, 5, 16, 16, 16)."""
    return join_protected_v1(MOE_TOP2_V1, [logits, top2_experts, requested_counts,
                                           admitted_counts, expert_offsets, route_slots,
                                           permutation, inverse], device, on_release)
