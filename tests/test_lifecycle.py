"""CPU tests of the exact LDS GEMM lifecycle (fe2o3_lds_gemm_slice1_*), the
mirror of crates/fe2o3-host/src/generated_lds_gemm_lifecycle.rs and its
tests (generated_lds_gemm_lifecycle_tests.rs:441-741).

No GPU is touched: the artifact, identities and join run on the host, and
load/dispatch/unload run against a Python adapter that records the order of
runtime events and substitutes one observation at a time (the reference's
fake adapter and its Fault list).  The buffers are host addresses; the
lifecycle only records them into the kernarg, and nothing dereferences them
here.  The HIP adapter itself runs in tests/test_gpu_lifecycle.py.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

from fe2o3_amd import _lib
from fe2o3_amd import lifecycle as lc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# ---- SHA-256 and the identities -----------------------------------------------------------

def test_sha256_known_answers_and_hashlib():
    # FIPS 180-4 examples (one block, two blocks) and the empty message
    assert lc.sha256(b"abc").hex() == (
        "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad")
    assert lc.sha256(b"").hex() == (
        "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855")
    assert lc.sha256(b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq").hex() == (
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1")
    rng = np.random.default_rng(1)
    for n in list(range(0, 130)) + [1000, 4095, 65537]:
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert lc.sha256(data) == hashlib.sha256(data).digest(), n


def _field(x: bytes) -> bytes:
    return struct.pack("<Q", len(x)) + x


def _length_identity(role, element, elements, nbytes):
    # lds_gemm_profile_registry.rs:672-690 framing
    h = hashlib.sha256()
    for f in (b"FE2O3/EXACT-LDS-GEMM-LENGTH/V1\0", bytes([role]), bytes([element]),
              struct.pack("<Q", elements), struct.pack("<Q", nbytes)):
        h.update(_field(f))
    return h.digest()


def test_buffer_contracts_and_length_identities():
    c = lc.artifact().contract
    expected = [(1, 1, 256, 512, 0, 0, 0), (2, 1, 256, 512, 0, 0, 0), (3, 2, 256, 1024, 1, 1, 1)]
    for buf, (role, element, n, nbytes, own, acc, alias) in zip(c.buffers, expected):
        assert (buf.role, buf.element, buf.elements, buf.bytes) == (role, element, n, nbytes)
        assert (buf.ownership, buf.access, buf.alias) == (own, acc, alias)
        assert bytes(buf.length_identity) == _length_identity(role, element, n, nbytes)


def test_profile_identity_framing():
    """The profile identity (lds_gemm_profile_registry.rs:606-660 framing)
    over the gfx950 contract."""
    c = lc.artifact().contract
    h = hashlib.sha256()
    h.update(_field(b"FE2O3/EXACT-LDS-GEMM-PROFILE/V1\0"))
    h.update(_field(bytes([1])))
    for f in (b"gfx950:xnack-", struct.pack("<H", 6), b"tiled_gemm_lds_slice1",
              b"tiled_gemm_lds_v1", b"tiled_gemm_lds_v1.kd", struct.pack("<I", 48),
              struct.pack("<I", 304), struct.pack("<I", 8), struct.pack("<3I", 1, 1, 1),
              struct.pack("<3I", 64, 1, 1), struct.pack("<I", 64), struct.pack("<I", 1024),
              struct.pack("<I", 2), struct.pack("<I", 512), struct.pack("<I", 16)):
        h.update(_field(f))
    for buf, tag in zip(c.buffers, (1, 1, 2)):
        for f in (bytes([buf.role]), struct.pack("<Q", buf.elements), struct.pack("<Q", buf.bytes),
                  bytes(buf.length_identity), bytes([tag])):
            h.update(_field(f))
    assert bytes(c.identity) == h.digest()
    assert bytes(lc.artifact().profile_identity) == h.digest()


# ---- the artifact --------------------------------------------------------------------------

def test_artifact_is_the_exact_cov6_abi():
    a = lc.artifact()
    i, c = a.inspection, a.contract
    assert bytes(a.finalizer_identity) == bytes(a.build_digest)
    built = os.path.join(ROOT, "fe2o3_amd", "csrc", "_build", "tiled_gemm_lds_v1.co")
    if os.path.exists(built):
        assert hashlib.sha256(open(built, "rb").read()).digest() == bytes(a.build_digest)
        assert os.path.getsize(built) == i.byte_len
    assert (c.target, c.code_object_version, c.profile) == (b"gfx950:xnack-", 6, 1)
    assert i.code_object_version == 6 and i.target == b"gfx950:xnack-"
    assert i.e_flags & 0xFF == 0x4F  # EF_AMDGPU_MACH_AMDGCN_GFX950
    assert (i.kd_kernarg_bytes, i.md_kernarg_bytes, i.md_kernarg_alignment) == (304, 304, 8)
    assert (i.explicit_args, i.explicit_bytes, i.implicit_offset, i.implicit_bytes) == (3, 48, 48, 256)
    assert (i.kd_group_segment_bytes, i.md_group_segment_bytes) == (1024, 1024)
    assert (i.kd_private_segment_bytes, i.md_private_segment_bytes) == (0, 0)
    assert (i.kd_wavefront_size, i.md_wavefront_size, i.md_max_flat_workgroup_size) == (64, 64, 64)
    assert (i.sgpr_spills, i.vgpr_spills, i.uses_dynamic_stack) == (0, 0, 0)
    assert (list(c.grid), list(c.workgroup), c.wavefront_size) == ([1, 1, 1], [64, 1, 1], 64)
    assert (c.explicit_kernarg_bytes, c.complete_kernarg_bytes, c.kernarg_alignment) == (48, 304, 8)
    assert (c.static_lds_bytes, c.lds_allocations, c.lds_bytes_per_allocation,
            c.lds_alignment) == (1024, 2, 512, 16)


# ---- join: every substitution is refused (lifecycle_tests.rs:441-487) ------------------------

def _m_buffer(attr, value):
    def f(x):
        setattr(x.contract.buffers[0], attr, value)
    return f


def _flip_length_identity(x):
    x.contract.buffers[0].length_identity[0] ^= 1


def _flip_host_length_identity(x):
    x.host_length_identities[0][0] ^= 1


def _set(attr, value):
    def f(x):
        setattr(x, attr, value)
    return f


def _set_contract(attr, value):
    def f(x):
        setattr(x.contract, attr, value)
    return f


def _set_index(obj_attr, index, value, contract=False):
    def f(x):
        getattr(x.contract if contract else x, obj_attr)[index] = value
    return f


MUTATIONS = {
    "ImportIdentity": (_set("import_matches", 0), ("ImportIdentity", "")),
    "ProfileIdentity": (_set("profile_matches", 0), ("ProfileIdentity", "")),
    "ContractBinding": (_set("contract_matches", 0), ("Contract", "")),
    "FinalizedOutput": (_set("finalized_output_matches", 0), ("FinalizedOutput", "digest")),
    "Inspection": (_set("inspection_matches", 0), ("FinalizedOutput", "code object inspection")),
    "Profile": (_set_contract("profile", 2), ("ContractField", "profile")),
    "Target": (_set_contract("target", b"gfx950:xnack+"), ("ContractField", "target")),
    "CodeObjectVersion": (_set_contract("code_object_version", 5),
                          ("ContractField", "code-object version")),
    "Grid": (_set_index("grid", 0, 2, True), ("ContractField", "grid")),
    "Workgroup": (_set_index("workgroup", 0, 256, True), ("ContractField", "workgroup")),
    "Wavefront": (_set_contract("wavefront_size", 32), ("ContractField", "wavefront")),
    "ExplicitKernarg": (_set_contract("explicit_kernarg_bytes", 40),
                        ("ContractField", "explicit kernarg size")),
    "CompleteKernarg": (_set_contract("complete_kernarg_bytes", 296),
                        ("ContractField", "complete kernarg size")),
    "ContractKernargAlignment": (_set_contract("kernarg_alignment", 16),
                                 ("ContractField", "descriptor kernarg alignment")),
    "StaticLds": (_set_contract("static_lds_bytes", 512), ("ContractField", "static LDS")),
    "LdsAllocations": (_set_contract("lds_allocations", 1), ("ContractField", "LDS allocation count")),
    "LdsBytesPerAllocation": (_set_contract("lds_bytes_per_allocation", 256),
                              ("ContractField", "LDS bytes per allocation")),
    "LdsAlignment": (_set_contract("lds_alignment", 8), ("ContractField", "LDS alignment")),
    "BufferRole": (_m_buffer("role", 2), ("BufferContract", "")),
    "BufferElement": (_m_buffer("element", 2), ("BufferContract", "")),
    "BufferElements": (_m_buffer("elements", 255), ("BufferContract", "")),
    "BufferBytes": (_m_buffer("bytes", 510), ("BufferContract", "")),
    "BufferLengthIdentity": (_flip_length_identity, ("BufferContract", "")),
    "BufferOwnership": (_m_buffer("ownership", 1), ("BufferContract", "")),
    "BufferAccess": (_m_buffer("access", 1), ("BufferContract", "")),
    "BufferAlias": (_m_buffer("alias", 1), ("BufferContract", "")),
    "HostTarget": (_set("host_target", b"gfx950:xnack+"), ("HostField", "target")),
    "HostProfile": (_set("host_profile", 2), ("HostField", "profile")),
    "HostProfileIdentity": (_set("host_profile_identity_matches", 0),
                            ("HostField", "profile identity")),
    "HostGrid": (_set_index("host_grid", 0, 2), ("HostField", "grid")),
    "HostWorkgroup": (_set_index("host_workgroup", 0, 256), ("HostField", "workgroup")),
    "HostStaticLds": (_set("host_static_lds", 512), ("HostField", "static LDS")),
    "HostDynamicLds": (_set("host_dynamic_lds", 1), ("HostField", "dynamic LDS")),
    "HostExplicitKernarg": (_set("host_explicit_kernarg", 40), ("HostField", "explicit kernarg size")),
    "HostCompleteKernarg": (_set("host_complete_kernarg", 296),
                            ("HostField", "complete kernarg size")),
    "HostContractKernargAlignment": (_set("host_kernarg_alignment", 16),
                                     ("HostField", "contract kernarg alignment")),
    "HostLengthIdentity": (_flip_host_length_identity, ("HostLengthIdentity", "")),
}


def test_canonical_join_facts_validate():
    f = lc.join_facts()
    assert all((f.import_matches, f.profile_matches, f.contract_matches,
                f.finalized_output_matches, f.inspection_matches,
                f.host_profile_identity_matches))
    lc.validate_join(f)


@pytest.mark.parametrize("name", list(MUTATIONS))
def test_join_rejects_substitution(name):
    mutate, (kind, field) = MUTATIONS[name]
    f = lc.join_facts()
    mutate(f)
    with pytest.raises(lc.JoinError) as e:
        lc.validate_join(f)
    assert (e.value.kind, e.value.field) == (kind, field), name
    if kind in ("BufferContract", "HostLengthIdentity"):
        assert e.value.index == 0


def test_join_reports_the_buffer_index():
    for i in range(3):
        f = lc.join_facts()
        f.contract.buffers[i].elements = 7
        with pytest.raises(lc.JoinError) as e:
            lc.validate_join(f)
        assert (e.value.kind, e.value.index) == ("BufferContract", i)
        f = lc.join_facts()
        f.host_length_identities[i][31] ^= 0x80
        with pytest.raises(lc.JoinError) as e:
            lc.validate_join(f)
        assert (e.value.kind, e.value.index) == ("HostLengthIdentity", i)


# ---- host-request preparation (generated_lds_gemm.rs:559-670) ---------------------------------

class Leases:
    def __init__(self):
        self.drops = 0

    def __call__(self):
        self.drops += 1


def _buffers():
    # one arena, regions 16 KiB apart: the overlap cases below cannot reach
    # a region other than the one they name, wherever the allocator puts it
    arena = np.zeros(3 * 16384, np.uint8)
    base = -arena.ctypes.data % 256
    a = arena[base:base + 512].view(np.uint16)
    b = arena[base + 16384:base + 16384 + 512].view(np.uint16)
    c = arena[base + 32768 - 256:base + 32768 - 256 + 1024].view(np.float32)
    return a, b, c


@pytest.mark.parametrize("case", ["a-length", "b-length", "c-length", "a-null", "c-null",
                                  "b-alignment", "c-alignment", "c-overlaps-a", "c-overlaps-b",
                                  "a-overflow"])
def test_host_request_preparation_rejects(case):
    a, b, c = _buffers()
    ra, rb, rc = (a.ctypes.data, 256), (b.ctypes.data, 256), (c.ctypes.data, 256)
    expect = {"a-length": ("Length", 0), "b-length": ("Length", 1), "c-length": ("Length", 2),
              "a-null": ("NullAddress", 0), "c-null": ("NullAddress", 2),
              "b-alignment": ("Alignment", 1), "c-alignment": ("Alignment", 2),
              "c-overlaps-a": ("OutputOverlap", 0), "c-overlaps-b": ("OutputOverlap", 1),
              "a-overflow": ("RegionAddressOverflow", 0)}[case]
    if case == "a-length":
        ra = (ra[0], 255)
    elif case == "b-length":
        rb = (rb[0], 257)
    elif case == "c-length":
        rc = (rc[0], 0)
    elif case == "a-null":
        ra = (0, 256)
    elif case == "c-null":
        rc = (0, 256)
    elif case == "b-alignment":
        rb = (rb[0] + 1, 256)
    elif case == "c-alignment":
        rc = (rc[0] + 2, 256)
    elif case == "c-overlaps-a":
        rc = (ra[0] + 4, 256)
    elif case == "c-overlaps-b":
        rc = (rb[0] - 1020, 256)
    elif case == "a-overflow":
        ra = (2**64 - 256, 256)
    leases = Leases()
    with pytest.raises(lc.JoinError) as e:
        lc.join_exact_lds_gemm_slice1_v1(ra, rb, rc, on_release=leases)
    assert (e.value.kind, e.value.index) == expect
    assert leases.drops == 1  # a refused join still releases its leases, once


def test_adjacent_regions_are_not_overlap():
    buf = np.zeros(512 + 256, np.float32)  # C right after B, sharing no byte
    base = buf.ctypes.data
    leases = Leases()
    j = lc.join_exact_lds_gemm_slice1_v1((base, 256), (base + 512, 256), (base + 1024, 256),
                                         on_release=leases)
    j.release()
    assert leases.drops == 1


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


class FakeAdapter(lc.RuntimeAdapter):
    """The reference's fake adapter (lifecycle_tests.rs:60-435): exact
    observations unless `fault` substitutes one."""

    def __init__(self, fault: str = "None", device: int = 0, context_ok: bool = True):
        self.fault, self.device, self.context_ok = fault, device, context_ok
        self.events: list[str] = []
        self.unloads = 0
        self.adapter_drops = 0
        self.aligned = False
        self.explicit_preserved = False
        self.hidden_initialized = False
        self.explicit = None

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
        _put(out.agent_runtime_instance,
             OTHER if self.fault == "EnvironmentRuntime" else RUNTIME)
        _put(out.agent_physical_uuid, OTHER if self.fault == "EnvironmentDevice" else UUID)
        return 0

    def load_executable(self, data, byte_len, digest, executable, out):
        self.events.append("load")
        if self.fault == "LoadAdapter":
            return 7
        blob = C.string_at(data, byte_len)
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
        assert executable == 0x1000 and symbol == b"tiled_gemm_lds_v1"
        if self.fault == "ResolveAdapter":
            return 9
        _put(out.executable_object, OTHER if self.fault == "ResolutionExecutable" else EXE)
        _put(out.kernel_object, KERNEL)
        out.symbol = b"tiled_gemm_lds_v2" if self.fault == "ResolutionSymbol" else symbol
        out.kernarg_segment_bytes = 296 if self.fault == "ResolutionSize" else 304
        out.kernarg_alignment = 8 if self.fault == "ResolutionAlignmentEight" else 16
        kernel[0] = 0x2000
        return 0

    def observe_resources(self, executable, kernel, out):
        self.events.append("resources")
        if self.fault == "ResourceAdapter":
            return 11
        _put(out.executable_object, OTHER if self.fault == "ResourceExecutable" else EXE)
        _put(out.kernel_object, OTHER if self.fault == "ResourceKernel" else KERNEL)
        out.group_segment_bytes = 512 if self.fault == "ResourceLds" else 1024
        out.private_segment_bytes = 1 if self.fault == "ResourcePrivate" else 0
        return 0

    def initialize_implicit_kernarg(self, executable, kernel, geometry, explicit_bytes,
                                    implicit_offset, implicit_bytes, kernarg, kernarg_bytes, out):
        self.events.append("implicit")
        self.aligned = C.addressof(kernarg.contents) % 16 == 0
        self.explicit = C.string_at(kernarg, 48)
        assert (explicit_bytes, implicit_offset, implicit_bytes, kernarg_bytes) == (48, 48, 256, 304)
        if self.fault == "ImplicitAdapter":
            return 13
        for i in range(implicit_offset, implicit_offset + implicit_bytes):
            kernarg[i] = 0
        kernarg[implicit_offset + 0] = geometry.grid[0]
        kernarg[implicit_offset + 12] = geometry.workgroup[0]
        self.hidden_initialized = True
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
        self.explicit_preserved = C.string_at(kernarg, 48) == self.explicit
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
        if self.fault == "UnloadAdapter":
            return 17
        _put(out.executable_object, EXE)
        _put(out.runtime_instance, RUNTIME)
        out.agent_handle = AGENT
        out.released = 0 if self.fault == "UnloadIncomplete" else 1
        return 0

    def drop_adapter(self):
        self.adapter_drops += 1


def _joined(leases):
    a, b, c = _buffers()
    j = lc.join_exact_lds_gemm_slice1_v1(a, b, c, on_release=leases)
    j._keep = (a, b, c)
    return j


def test_successful_lifecycle_has_exact_order_alignment_spans_and_retention():
    fake, leases = FakeAdapter(), Leases()
    joined = _joined(leases)
    a, b, c = joined._keep
    loaded = joined.load(fake)
    assert leases.drops == 0
    assert fake.events == ["environment", "load", "resolve", "resources"]
    obs = loaded.observation()
    assert obs.state == lc.LOADED and obs.leases_retained and obs.holds_executable
    assert obs.resolution.kernarg_segment_bytes == 304 and obs.resources.group_segment_bytes == 1024

    completed = loaded.dispatch_and_wait()
    # quiescent completion releases the joined request and the A/B/C leases;
    # the executable stays loaded until unload
    assert leases.drops == 1 and fake.unloads == 0
    assert fake.aligned and fake.explicit_preserved and fake.hidden_initialized
    # the explicit prefix: {address, 256} for A, B, C, little-endian
    assert fake.explicit == struct.pack("<6Q", a.ctypes.data, 256, b.ctypes.data, 256,
                                        c.ctypes.data, 256)
    obs = completed.observation()
    assert obs.state == lc.COMPLETED and not obs.leases_retained and not obs.holds_kernel
    assert completed.dispatch_identity == DISPATCH

    receipt = completed.unload()
    assert (receipt.executable_object, receipt.kernel_object, receipt.dispatch_identity) == (
        EXE, KERNEL, DISPATCH)
    h = hashlib.sha256()
    for f in (b"FE2O3/EXACT-LDS-GEMM/UNLOAD/V1\0", EXE, RUNTIME, struct.pack("<Q", AGENT),
              bytes([1])):
        h.update(_field(f))
    assert receipt.unload_identity == h.digest()
    art = lc.artifact()
    assert receipt.finalizer_identity == bytes(art.finalizer_identity)
    assert receipt.profile_identity == bytes(art.profile_identity)
    assert receipt.import_identity == bytes(art.import_identity)
    assert leases.drops == 1 and fake.unloads == 1 and fake.adapter_drops == 1
    assert fake.events == ["environment", "load", "resolve", "resources", "implicit",
                           "dispatch", "kernel_drop", "unload"]


def test_context_and_environment_rejections_create_no_native_authority():
    fake, leases = FakeAdapter(context_ok=False), Leases()
    with pytest.raises(lc.LoadError) as e:
        _joined(leases).load(fake)
    assert e.value.kind == "ContextIdentity"
    assert fake.events == [] and fake.unloads == 0 and leases.drops == 1
    assert fake.adapter_drops == 1
    for fault, kind, field in [("EnvironmentAdapter", "EnvironmentAdapter", ""),
                               ("EnvironmentTarget", "Environment", "physical-device target"),
                               ("EnvironmentOrdinal", "Environment", "HIP ordinal"),
                               ("EnvironmentRuntime", "Environment", "runtime instance"),
                               ("EnvironmentDevice", "Environment", "physical device"),
                               ("LoadAdapter", "LoadAdapter", "")]:
        fake, leases = FakeAdapter(fault), Leases()
        with pytest.raises(lc.LoadError) as e:
            _joined(leases).load(fake)
        assert (e.value.kind, e.value.field) == (kind, field), fault
        assert fake.unloads == 0 and leases.drops == 1 and fake.adapter_drops == 1, fault
    assert e.value.adapter_status == 7


@pytest.mark.parametrize("fault,kind", [
    ("LoadDigest", "LoadObservation"), ("LoadLength", "LoadObservation"),
    ("LoadRuntime", "LoadObservation"), ("LoadAgent", "LoadObservation"),
    ("ResolveAdapter", "KernelAdapter"), ("ResolutionExecutable", "KernelObservation"),
    ("ResolutionSymbol", "KernelObservation"), ("ResolutionSize", "KernelObservation"),
    ("ResolutionAlignmentEight", "KernelObservation")])
def test_load_and_resolution_substitutions_cleanup_exactly_once(fault, kind):
    fake, leases = FakeAdapter(fault), Leases()
    with pytest.raises(lc.LoadError) as e:
        _joined(leases).load(fake)
    assert e.value.kind == kind
    assert fake.unloads == 1 and leases.drops == 1 and fake.adapter_drops == 1
    assert fake.events[-1] == "unload"
    if "kernel_drop" in fake.events:
        assert fake.events.index("kernel_drop") < fake.events.index("unload")


@pytest.mark.parametrize("fault,kind", [
    ("ResourceAdapter", "ResourceAdapter"), ("ResourceExecutable", "ResourceObservation"),
    ("ResourceKernel", "ResourceObservation"), ("ResourceLds", "ResourceObservation"),
    ("ResourcePrivate", "ResourceObservation")])
def test_runtime_resource_substitutions_cleanup_exactly_once(fault, kind):
    fake, leases = FakeAdapter(fault), Leases()
    with pytest.raises(lc.LoadError) as e:
        _joined(leases).load(fake)
    assert e.value.kind == kind
    assert fake.unloads == 1 and leases.drops == 1
    assert fake.events.index("kernel_drop") < fake.events.index("unload")


@pytest.mark.parametrize("fault,kind", [
    ("ImplicitAdapter", "ImplicitAdapter"), ("ImplicitExecutable", "ImplicitObservation"),
    ("ImplicitKernel", "ImplicitObservation"), ("ImplicitGeometry", "ImplicitObservation"),
    ("ImplicitSpan", "ImplicitObservation"), ("ImplicitIncomplete", "ImplicitObservation"),
    ("ExplicitMutation", "ExplicitKernargMutation"), ("DispatchAdapter", "DispatchAdapter"),
    ("DispatchExecutable", "DispatchObservation"), ("DispatchKernel", "DispatchObservation"),
    ("DispatchGeometry", "DispatchObservation"), ("DispatchIncomplete", "DispatchObservation")])
def test_implicit_and_dispatch_failures_are_recoverable_only_with_terminal_cleanup(fault, kind):
    fake, leases = FakeAdapter(fault), Leases()
    loaded = _joined(leases).load(fake)
    with pytest.raises(lc.DispatchError) as e:
        loaded.dispatch_and_wait()
    assert e.value.kind == kind
    assert fake.unloads == 1 and leases.drops == 1 and fake.adapter_drops == 1
    assert fake.events.index("kernel_drop") < fake.events.index("unload")


def test_dropping_loaded_or_completed_state_unloads_once():
    fake, leases = FakeAdapter(), Leases()
    loaded = _joined(leases).load(fake)
    loaded.release()
    assert fake.unloads == 1 and leases.drops == 1 and fake.adapter_drops == 1
    assert fake.events == ["environment", "load", "resolve", "resources", "kernel_drop", "unload"]
    fake, leases = FakeAdapter(), Leases()
    completed = _joined(leases).load(fake).dispatch_and_wait()
    del completed  # Drop
    assert fake.unloads == 1 and leases.drops == 1 and fake.adapter_drops == 1
    # a joined request dropped before load releases its leases and nothing else
    leases = Leases()
    _joined(leases).release()
    assert leases.drops == 1


def test_consumed_values_and_out_of_order_calls_are_refused():
    fake, leases = FakeAdapter(), Leases()
    joined = _joined(leases)
    loaded = joined.load(fake)
    with pytest.raises(lc.StateError):
        joined.load(FakeAdapter())
    completed = loaded.dispatch_and_wait()
    with pytest.raises(lc.StateError):
        loaded.dispatch_and_wait()
    completed.unload()
    with pytest.raises(lc.StateError):
        completed.unload()
    # the C-ABI refuses a transition from the wrong state and changes nothing
    L = _lib.lib()
    a, b, c = _buffers()
    out = C.c_void_p()
    err = _lib.Fe2o3Slice1ErrorV1()
    assert L.fe2o3_lds_gemm_slice1_join_v1(a.ctypes.data, 256, b.ctypes.data, 256, c.ctypes.data,
                                           256, 0, _lib.SLICE1_RELEASE_FN(0), None, C.byref(out),
                                           C.byref(err)) == 0
    assert L.fe2o3_lds_gemm_slice1_dispatch_and_wait_v1(out, C.byref(err)) == lc.ERR_STATE
    receipt = _lib.Fe2o3Slice1ReceiptV1()
    assert L.fe2o3_lds_gemm_slice1_unload_v1(out, C.byref(receipt)) == lc.ERR_STATE
    obs = _lib.Fe2o3Slice1ObservationV1()
    assert L.fe2o3_lds_gemm_slice1_observe_v1(out, C.byref(obs)) == 0
    assert obs.state == lc.JOINED and obs.leases_retained
    L.fe2o3_lds_gemm_slice1_release_v1(out)


_CHILD = r"""
import sys
sys.path[:0] = [{root!r}, {tests!r}]
import test_lifecycle as t
fake = t.FakeAdapter({fault!r})
loaded = t._joined(t.Leases()).load(fake)
loaded.release()
print("unreachable", flush=True)
"""


@pytest.mark.parametrize("fault", ["UnloadAdapter", "UnloadIncomplete"])
def test_unload_ambiguity_is_process_terminal(fault):
    """lifecycle_tests.rs:700-741: an unload that fails or is not confirmed
    ends the process (SIGABRT), in a child process."""
    code = _CHILD.format(root=ROOT, tests=os.path.join(ROOT, "tests"), fault=fault)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == -6, (r.returncode, r.stdout, r.stderr)
    assert "unreachable" not in r.stdout
