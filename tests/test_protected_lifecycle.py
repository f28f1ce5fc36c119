"""CPU tests of the protected profile lifecycles (fe2o3_protected_*): the
flash-attention, row-softmax and top-2 routing profiles, mirrors of
crates/fe2o3-host/src/flash_attention_v1_lifecycle.rs,
protected_row_softmax_v1_lifecycle.rs and moe_top2_v1_lifecycle.rs and of
their tests (flash_attention_v1_lifecycle_tests.rs:451-592 and the two
siblings: exact order and ABI, every load/resource substitution failing
closed with exact cleanup, implicit and dispatch failures, drop while loaded
or completed).

No GPU is touched: the artifacts, identities and join run on the host, and
load/dispatch/unload run against a Python adapter that records the order of
runtime events and substitutes one observation at a time.  The regions are
host addresses that only go into the kernarg.  The HIP adapter runs these
lifecycles in tests/test_gpu_protected_lifecycle.py.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import struct

import numpy as np
import pytest

from fe2o3_amd import _lib
from fe2o3_amd import lifecycle as lc

# the reference's profile constants (…_lifecycle.rs:20-32 of each file)
PROFILES = {
    lc.FLASH_ATTENTION_V1: dict(
        symbol=b"flash_attention_causal_f32_b1_h1_n8_d16_v1", explicit=64, complete=320,
        elements=[128, 128, 128, 128], writes=[0, 0, 0, 1], shape=[1, 1, 8, 16],
        unload_domain=b"FE2O3/FLASH-ATTENTION/UNLOAD/V1\0",
        receipt=["identity", "artifact identity", "finalized output", "raw worker output",
                 "target", "code-object version", "frontend authority commitment",
                 "OCML provider commitment", "finalization", "compiler handoff",
                 "machine identity", "OCML provider closure"],
        host=["target", "shape", "argument extent", "grid", "workgroup", "code-object version",
              "explicit ABI", "complete ABI", "ABI alignment", "mask policy"]),
    lc.ROW_SOFTMAX_V1: dict(
        symbol=b"row_softmax_v1", explicit=32, complete=288, elements=[64, 64], writes=[0, 1],
        shape=[64, 0, 0, 0], unload_domain=b"FE2O3/ROW-SOFTMAX/UNLOAD/V1\0",
        receipt=["identity", "admission identity", "artifact identity", "finalized output",
                 "target", "row width", "grid", "workgroup", "explicit ABI", "complete ABI"],
        host=["target", "row width", "grid", "workgroup", "explicit ABI", "complete ABI",
              "ABI alignment", "activity policy"]),
    lc.MOE_TOP2_V1: dict(
        symbol=b"moe_top2_route_f32_t8_e4_k2_c4_v1", explicit=128, complete=384,
        elements=[32, 16, 4, 4, 5, 16, 16, 16], writes=[0, 1, 1, 1, 1, 1, 1, 1],
        shape=[8, 4, 2, 4], unload_domain=b"FE2O3/MOE-TOP2/UNLOAD/V1\0",
        receipt=["identity", "artifact identity", "finalized output", "raw worker output",
                 "target", "code-object version", "canonical digest",
                 "source/KIR/compiler profile", "upstream LLVM/LLD exchange"],
        host=["target", "T/E/K/C profile", "grid", "workgroup", "code-object version",
              "explicit ABI", "complete ABI", "ABI alignment", "routing-only policy"]),
}
IDS = {lc.FLASH_ATTENTION_V1: "flash", lc.ROW_SOFTMAX_V1: "softmax", lc.MOE_TOP2_V1: "moe"}
ALL = pytest.mark.parametrize("profile", list(PROFILES), ids=[IDS[p] for p in PROFILES])


def _field(x: bytes) -> bytes:
    return struct.pack("<Q", len(x)) + x


def _sha(*fields: bytes) -> bytes:
    h = hashlib.sha256()
    for f in fields:
        h.update(_field(f))
    return h.digest()


class Leases:
    def __init__(self):
        self.drops = 0

    def __call__(self):
        self.drops += 1


def _regions(profile):
    """Disjoint host regions of the profile's lengths (4-byte elements)."""
    p = PROFILES[profile]
    bufs = [np.zeros(n, np.float32) for n in p["elements"]]
    return bufs


# ---- the profile and its artifact ------------------------------------------------------------

@ALL
def test_profile_facts_are_the_references(profile):
    p, v = PROFILES[profile], lc.protected_profile(profile)
    assert v.symbol == p["symbol"] and v.target == b"gfx950:xnack-"
    assert v.code_object_version == 6
    assert list(v.grid) == [1, 1, 1] and list(v.workgroup) == [64, 1, 1]
    assert (v.dynamic_lds_bytes, v.static_lds_bytes, v.private_segment_bytes) == (0, 0, 0)
    assert (v.explicit_kernarg_bytes, v.complete_kernarg_bytes) == (p["explicit"], p["complete"])
    assert (v.kernarg_alignment, v.hsa_kernarg_alignment) == (8, 16)
    assert v.regions == len(p["elements"]) and v.explicit_kernarg_bytes == 16 * v.regions
    assert list(v.region_elements)[:v.regions] == p["elements"]
    assert list(v.region_element_bytes)[:v.regions] == [4] * v.regions
    assert list(v.region_writes)[:v.regions] == p["writes"]
    assert list(v.shape) == p["shape"]
    assert [v.receipt_field[i].value.decode() for i in range(v.receipt_fields)] == p["receipt"]
    assert [v.host_field[i].value.decode() for i in range(v.host_fields)] == p["host"]


@ALL
def test_artifact_is_the_exact_cov6_object_and_identities_are_framed(profile):
    p, a = PROFILES[profile], lc.protected_artifact(profile)
    i = a.inspection
    assert i.code_object_version == 6 and i.target == b"gfx950:xnack-"
    assert (i.e_flags & 0xFF) == 0x4F  # EF_AMDGPU_MACH_AMDGCN_GFX950
    assert i.kd_kernarg_bytes == i.md_kernarg_bytes == p["complete"]
    assert i.explicit_bytes == p["explicit"] and i.explicit_args == len(p["elements"])
    assert i.implicit_offset == p["explicit"] and i.implicit_bytes == p["complete"] - p["explicit"]
    assert i.kd_group_segment_bytes == i.md_group_segment_bytes == 0
    assert i.kd_private_segment_bytes == i.md_private_segment_bytes == 0
    assert (i.sgpr_spills, i.vgpr_spills, i.uses_dynamic_stack) == (0, 0, 0)
    assert i.md_wavefront_size == 64 and i.md_max_flat_workgroup_size == 64
    assert bytes(a.artifact_identity) == bytes(a.build_digest)
    # profile identity over the profile's facts, receipt identity over the
    # four artifact identities (length-prefixed fields, NUL-terminated domains)
    v = a.profile
    fields = [b"FE2O3/MI355X-PROTECTED-PROFILE/V1\0", struct.pack("<I", profile), v.name,
              b"gfx950:xnack-", v.symbol] + [struct.pack("<I", 1)] * 3 + \
        [struct.pack("<I", 64), struct.pack("<I", 1), struct.pack("<I", 1),
         struct.pack("<I", p["explicit"]), struct.pack("<I", p["complete"])]
    for n, w in zip(p["elements"], p["writes"]):
        fields += [struct.pack("<Q", n), struct.pack("<I", 4), struct.pack("<I", w)]
    fields += [struct.pack("<I", s) for s in p["shape"]]
    assert bytes(a.profile_identity) == _sha(*fields)
    assert bytes(a.identity) == _sha(b"FE2O3/MI355X-PROTECTED-RECEIPT/V1\0",
                                     bytes(a.profile_identity), bytes(a.artifact_identity),
                                     bytes(a.source_digest), bytes(a.compiler_identity))


# ---- join ----------------------------------------------------------------------------------------

@ALL
def test_canonical_join_facts_validate(profile):
    f = lc.protected_join_facts(profile)
    n = len(PROFILES[profile]["receipt"])
    assert list(f.receipt)[:n] == [1] * n
    lc.protected_validate_join(f)


@ALL
def test_each_receipt_field_is_checked_in_order(profile):
    names = PROFILES[profile]["receipt"]
    for i, name in enumerate(names):
        f = lc.protected_join_facts(profile)
        f.receipt[i] = 0
        with pytest.raises(lc.JoinError) as e:
            lc.protected_validate_join(f)
        assert (e.value.kind, e.value.field) == ("ReceiptField", name)
        # with a later field broken too, the earlier one is reported
        if i + 1 < len(names):
            f.receipt[len(names) - 1] = 0
            with pytest.raises(lc.JoinError) as e:
                lc.protected_validate_join(f)
            assert e.value.field == name


def _break_host(f, name):
    if name == "target":
        f.host_target = b"gfx942:xnack-"
    elif name in ("shape", "row width", "T/E/K/C profile"):
        f.host_shape[0] += 1
    elif name == "argument extent":
        f.host_argument_elements -= 1
    elif name == "grid":
        f.host_grid[2] = 2
    elif name == "workgroup":
        f.host_workgroup[0] = 32
    elif name == "code-object version":
        f.host_code_object_version = 5
    elif name == "explicit ABI":
        f.host_explicit_kernarg += 8
    elif name == "complete ABI":
        f.host_complete_kernarg -= 8
    elif name == "ABI alignment":
        f.host_kernarg_alignment = 16
    else:
        f.host_policy = 0


@ALL
def test_each_host_field_is_checked_in_order(profile):
    names = PROFILES[profile]["host"]
    for i, name in enumerate(names):
        f = lc.protected_join_facts(profile)
        _break_host(f, name)
        for later in names[i + 1:]:
            _break_host(f, later)
        with pytest.raises(lc.JoinError) as e:
            lc.protected_validate_join(f)
        assert (e.value.kind, e.value.field) == ("HostField", name)
    # receipt fields come before host fields
    f = lc.protected_join_facts(profile)
    _break_host(f, names[0])
    f.receipt[0] = 0
    with pytest.raises(lc.JoinError) as e:
        lc.protected_validate_join(f)
    assert e.value.kind == "ReceiptField"


@ALL
def test_host_request_preparation_rejects(profile):
    p = PROFILES[profile]
    n = len(p["elements"])
    for role in range(n):
        bufs = _regions(profile)
        regions = [(b.ctypes.data, b.size) for b in bufs]
        # length
        bad = list(regions)
        bad[role] = (bad[role][0], bad[role][1] - 1)
        leases = Leases()
        with pytest.raises(lc.JoinError) as e:
            lc.join_protected_v1(profile, bad, on_release=leases)
        assert (e.value.kind, e.value.index) == ("Length", role)
        assert (e.value.expected, e.value.actual) == (p["elements"][role], p["elements"][role] - 1)
        assert leases.drops == 1  # released also when refused
        # null
        bad = list(regions)
        bad[role] = (0, bad[role][1])
        with pytest.raises(lc.JoinError) as e:
            lc.join_protected_v1(profile, bad)
        assert (e.value.kind, e.value.index) == ("NullAddress", role)
        # alignment (4-byte elements)
        big = np.zeros(256, np.float32)
        bad = list(regions)
        bad[role] = (big.ctypes.data + 2, bad[role][1])
        with pytest.raises(lc.JoinError) as e:
            lc.join_protected_v1(profile, bad)
        assert (e.value.kind, e.value.index, e.value.expected) == ("Alignment", role, 4)
        # address overflow
        bad = list(regions)
        bad[role] = (2**64 - 8, bad[role][1])
        with pytest.raises(lc.JoinError) as e:
            lc.join_protected_v1(profile, bad)
        assert (e.value.kind, e.value.index) == ("RegionAddressOverflow", role)
    # region count
    bufs = _regions(profile)
    with pytest.raises(lc.JoinError) as e:
        lc.join_protected_v1(profile, [(b.ctypes.data, b.size) for b in bufs][:-1])
    assert e.value.kind == "Length" and e.value.index == -1


@ALL
def test_written_regions_overlap_nothing_and_inputs_may_alias(profile):
    p = PROFILES[profile]
    n = len(p["elements"])
    arena = np.zeros(4096, np.float32)
    base = arena.ctypes.data
    for left in range(n):
        for right in range(left + 1, n):
            # every region its own 1 KiB slot, then `right` moved onto `left`
            regions = [(base + 1024 * i, p["elements"][i]) for i in range(n)]
            regions[right] = (regions[left][0], p["elements"][right])
            if p["writes"][left] or p["writes"][right]:
                with pytest.raises(lc.JoinError) as e:
                    lc.join_protected_v1(profile, regions)
                assert (e.value.kind, e.value.index, e.value.actual) == ("OutputOverlap", left, right)
            elif p["elements"][left] == p["elements"][right]:
                lc.join_protected_v1(profile, regions).release()
    # regions that only touch are not an overlap
    regions, at = [], base
    for e in p["elements"]:
        regions.append((at, e))
        at += 4 * e
    lc.join_protected_v1(profile, regions).release()


# ---- the fake runtime adapter ------------------------------------------------------------------

RUNTIME = bytes(range(16))
UUID = bytes(range(100, 116))
AGENT = 0x0000_0001_0000_4200
EXE = bytes([0xE1] * 16)
KERNEL = bytes([0x4B] * 16)
DISPATCH = bytes([0xD1] * 16)
OTHER = bytes([0x99] * 16)


def _put(arr, data: bytes):
    for i, v in enumerate(data):
        arr[i] = v


class ProtectedFake(lc.RuntimeAdapter):
    """The reference's fake adapter (flash_attention_v1_lifecycle_tests.rs:
    149-435) for one profile: exact observations unless `fault` substitutes
    one."""

    def __init__(self, profile, fault: str = "None", device: int = 0, context_ok: bool = True):
        self.p = PROFILES[profile]
        self.fault, self.device, self.context_ok = fault, device, context_ok
        self.events: list[str] = []
        self.unloads = 0
        self.adapter_drops = 0
        self.explicit = None
        self.explicit_preserved = False
        self.loaded_bytes = None

    def context_identity(self, identity):
        _put(identity, lc.context_identity(self.device) if self.context_ok else bytes(16))
        return 0

    def observe_environment(self, out):
        self.events.append("environment")
        if self.fault == "EnvironmentAdapter":
            return 5
        _put(out.runtime_instance, RUNTIME)
        target = b"gfx942:xnack-" if self.fault == "EnvironmentTarget" else b"gfx950:sramecc+:xnack-"
        out.physical_target = target
        out.agent_target = target
        out.hip_ordinal = self.device + (1 if self.fault == "EnvironmentOrdinal" else 0)
        _put(out.physical_uuid, UUID)
        out.agent_handle = AGENT
        _put(out.agent_runtime_instance, OTHER if self.fault == "EnvironmentRuntime" else RUNTIME)
        _put(out.agent_physical_uuid, OTHER if self.fault == "EnvironmentDevice" else UUID)
        return 0

    def load_executable(self, data, byte_len, digest, executable, out):
        self.events.append("load")
        if self.fault == "LoadAdapter":
            return 7
        blob = C.string_at(data, byte_len)
        self.loaded_bytes = blob
        d = hashlib.sha256(blob).digest()
        assert bytes(digest) == d
        _put(out.digest, bytes([d[0] ^ 1]) + d[1:] if self.fault == "LoadDigest" else d)
        out.byte_len = byte_len + (1 if self.fault == "LoadLength" else 0)
        _put(out.runtime_instance, OTHER if self.fault == "LoadRuntime" else RUNTIME)
        out.agent_handle = AGENT + (1 if self.fault == "LoadAgent" else 0)
        _put(out.executable_object, EXE)
        executable[0] = 0x1000
        return 0

    def resolve_kernel(self, executable, symbol, kernel, out):
        self.events.append("resolve")
        assert executable == 0x1000 and symbol == self.p["symbol"]
        if self.fault == "ResolveAdapter":
            return 9
        _put(out.executable_object, OTHER if self.fault == "ResolutionExecutable" else EXE)
        _put(out.kernel_object, KERNEL)
        out.symbol = symbol + b"_v2" if self.fault == "ResolutionSymbol" else symbol
        out.kernarg_segment_bytes = self.p["complete"] - (8 if self.fault == "ResolutionSize" else 0)
        out.kernarg_alignment = 8 if self.fault == "ResolutionAlignmentEight" else 16
        kernel[0] = 0x2000
        return 0

    def observe_resources(self, executable, kernel, out):
        self.events.append("resources")
        if self.fault == "ResourceAdapter":
            return 11
        _put(out.executable_object, OTHER if self.fault == "ResourceExecutable" else EXE)
        _put(out.kernel_object, OTHER if self.fault == "ResourceKernel" else KERNEL)
        out.group_segment_bytes = 16 if self.fault == "ResourceLds" else 0
        out.private_segment_bytes = 1 if self.fault == "ResourcePrivate" else 0
        return 0

    def initialize_implicit_kernarg(self, executable, kernel, geometry, explicit_bytes,
                                    implicit_offset, implicit_bytes, kernarg, kernarg_bytes, out):
        self.events.append("implicit")
        e, c = self.p["explicit"], self.p["complete"]
        self.aligned = C.addressof(kernarg.contents) % 16 == 0
        self.explicit = C.string_at(kernarg, e)
        assert (explicit_bytes, implicit_offset, implicit_bytes, kernarg_bytes) == (e, e, c - e, c)
        if self.fault == "ImplicitAdapter":
            return 13
        for i in range(implicit_offset, implicit_offset + implicit_bytes):
            kernarg[i] = 0
        kernarg[implicit_offset + 0] = geometry.grid[0]
        kernarg[implicit_offset + 12] = geometry.workgroup[0]
        if self.fault == "ExplicitMutation":
            kernarg[3] ^= 1
        _put(out.executable_object, OTHER if self.fault == "ImplicitExecutable" else EXE)
        _put(out.kernel_object, OTHER if self.fault == "ImplicitKernel" else KERNEL)
        C.memmove(C.addressof(out.geometry), C.addressof(geometry), C.sizeof(geometry))
        if self.fault == "ImplicitGeometry":
            out.geometry.grid[0] = 2
        out.explicit_bytes, out.implicit_offset = explicit_bytes, implicit_offset
        out.implicit_bytes = implicit_bytes - (1 if self.fault == "ImplicitSpan" else 0)
        out.completed = 0 if self.fault == "ImplicitIncomplete" else 1
        return 0

    def launch_and_wait(self, executable, kernel, geometry, kernarg, kernarg_bytes, out):
        self.events.append("dispatch")
        self.explicit_preserved = C.string_at(kernarg, self.p["explicit"]) == self.explicit
        if self.fault == "DispatchAdapter":
            return 15
        _put(out.dispatch_identity, DISPATCH)
        _put(out.executable_object, OTHER if self.fault == "DispatchExecutable" else EXE)
        _put(out.kernel_object, OTHER if self.fault == "DispatchKernel" else KERNEL)
        C.memmove(C.addressof(out.geometry), C.addressof(geometry), C.sizeof(geometry))
        if self.fault == "DispatchGeometry":
            out.geometry.workgroup[0] = 32
        out.completed = 0 if self.fault == "DispatchIncomplete" else 1
        return 0

    def drop_kernel(self, kernel):
        assert kernel == 0x2000
        self.events.append("kernel_drop")

    def unload_executable(self, executable, out):
        assert executable == 0x1000
        self.events.append("unload")
        self.unloads += 1
        _put(out.executable_object, EXE)
        _put(out.runtime_instance, RUNTIME)
        out.agent_handle = AGENT
        out.released = 1
        return 0

    def drop_adapter(self):
        self.adapter_drops += 1


def _joined(profile, leases):
    bufs = _regions(profile)
    j = lc.join_protected_v1(profile, bufs, on_release=leases)
    j._keep = bufs
    return j


@ALL
def test_successful_lifecycle_has_exact_order_abi_and_releases_leases_at_quiescence(profile):
    p = PROFILES[profile]
    fake, leases = ProtectedFake(profile), Leases()
    joined = _joined(profile, leases)
    bufs = joined._keep
    loaded = joined.load(fake)
    assert fake.events == ["environment", "load", "resolve", "resources"]
    assert fake.loaded_bytes is not None
    assert hashlib.sha256(fake.loaded_bytes).digest() == joined.artifact_identity
    assert leases.drops == 0
    completed = loaded.dispatch_and_wait()
    assert fake.events[4:] == ["implicit", "dispatch", "kernel_drop"]
    assert fake.aligned and fake.explicit_preserved
    # the explicit kernarg: one {address, elements} per region in role order
    expected = b"".join(struct.pack("<QQ", b.ctypes.data, b.size) for b in bufs)
    assert fake.explicit == expected and len(expected) == p["explicit"]
    assert leases.drops == 1  # quiescent: the regions are released
    assert completed.dispatch_identity == DISPATCH
    receipt = completed.unload()
    assert fake.events[-1] == "unload" and fake.unloads == 1 and fake.adapter_drops == 1
    assert receipt.profile == profile and receipt.executable_object == EXE
    assert receipt.kernel_object == KERNEL and receipt.dispatch_identity == DISPATCH
    assert receipt.identity == joined.identity
    assert receipt.unload_identity == _sha(p["unload_domain"], EXE, RUNTIME,
                                           struct.pack("<Q", AGENT), b"\x01")
    with pytest.raises(lc.StateError):
        completed.unload()


LOAD_FAULTS = [
    ("EnvironmentAdapter", "EnvironmentAdapter", False), ("EnvironmentTarget", "Environment", False),
    ("EnvironmentOrdinal", "Environment", False), ("EnvironmentRuntime", "Environment", False),
    ("EnvironmentDevice", "Environment", False), ("LoadAdapter", "LoadAdapter", False),
    ("LoadDigest", "LoadObservation", True), ("LoadLength", "LoadObservation", True),
    ("LoadRuntime", "LoadObservation", True), ("LoadAgent", "LoadObservation", True),
    ("ResolveAdapter", "KernelAdapter", True), ("ResolutionExecutable", "KernelObservation", True),
    ("ResolutionSymbol", "KernelObservation", True), ("ResolutionSize", "KernelObservation", True),
    ("ResolutionAlignmentEight", "KernelObservation", True),
    ("ResourceAdapter", "ResourceAdapter", True), ("ResourceExecutable", "ResourceObservation", True),
    ("ResourceKernel", "ResourceObservation", True), ("ResourceLds", "ResourceObservation", True),
    ("ResourcePrivate", "ResourceObservation", True),
]


@ALL
@pytest.mark.parametrize("fault,kind,unloads", LOAD_FAULTS, ids=[f[0] for f in LOAD_FAULTS])
def test_every_load_and_resource_substitution_fails_closed_with_exact_cleanup(profile, fault, kind,
                                                                              unloads):
    fake, leases = ProtectedFake(profile, fault), Leases()
    joined = _joined(profile, leases)
    with pytest.raises(lc.LoadError) as e:
        joined.load(fake)
    assert e.value.kind == kind
    assert fake.unloads == (1 if unloads else 0)
    assert ("kernel_drop" in fake.events) == (kind in ("KernelObservation", "ResourceAdapter",
                                                        "ResourceObservation"))
    assert leases.drops == 1 and fake.adapter_drops == 1


DISPATCH_FAULTS = [
    ("ImplicitAdapter", "ImplicitAdapter"), ("ExplicitMutation", "ExplicitKernargMutation"),
    ("ImplicitExecutable", "ImplicitObservation"), ("ImplicitKernel", "ImplicitObservation"),
    ("ImplicitGeometry", "ImplicitObservation"), ("ImplicitSpan", "ImplicitObservation"),
    ("ImplicitIncomplete", "ImplicitObservation"), ("DispatchAdapter", "DispatchAdapter"),
    ("DispatchExecutable", "DispatchObservation"), ("DispatchKernel", "DispatchObservation"),
    ("DispatchGeometry", "DispatchObservation"), ("DispatchIncomplete", "DispatchObservation"),
]


@ALL
@pytest.mark.parametrize("fault,kind", DISPATCH_FAULTS, ids=[f[0] for f in DISPATCH_FAULTS])
def test_implicit_and_dispatch_failures_cleanup_once(profile, fault, kind):
    fake, leases = ProtectedFake(profile, fault), Leases()
    loaded = _joined(profile, leases).load(fake)
    with pytest.raises(lc.DispatchError) as e:
        loaded.dispatch_and_wait()
    assert e.value.kind == kind
    assert fake.events[-2:] == ["kernel_drop", "unload"] and fake.unloads == 1
    assert leases.drops == 1 and fake.adapter_drops == 1


@ALL
def test_dropping_loaded_or_completed_state_unloads_exactly_once(profile):
    for advance in (False, True):
        fake, leases = ProtectedFake(profile), Leases()
        state = _joined(profile, leases).load(fake)
        if advance:
            state = state.dispatch_and_wait()
        state.release()
        state.release()
        assert fake.unloads == 1 and fake.adapter_drops == 1 and leases.drops == 1
        assert fake.events.count("kernel_drop") == 1


@ALL
def test_context_mismatch_and_cross_family_calls_are_refused(profile):
    fake, leases = ProtectedFake(profile, context_ok=False), Leases()
    with pytest.raises(lc.LoadError) as e:
        _joined(profile, leases).load(fake)
    assert e.value.kind == "ContextIdentity" and fake.events == []
    assert leases.drops == 1 and fake.adapter_drops == 1
    # a protected handle is not an LDS GEMM handle, nor the reverse
    j = _joined(profile, Leases())
    L = _lib.lib()
    err = _lib.Fe2o3Slice1ErrorV1()
    table = ProtectedFake(profile).table()
    assert L.fe2o3_lds_gemm_slice1_load_v1(j._handle.ptr, C.byref(table), C.byref(err)) == \
        lc.ERR_STATE
    j.release()
