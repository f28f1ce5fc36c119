"""CPU checks of the C-ABI boundary: the library loads (no GPU calls), exports
every function include/fe2o3_mi355x.h declares, the ctypes table covers the
same set, the 312-byte property record layout matches
crates/fe2o3-hip-sys/src/lib.rs:190-214, and host-side validation fails
closed before any launch."""
from __future__ import annotations

import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    with open(os.path.join(ROOT, "include", "fe2o3_mi355x.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fe2o3\w+|fe2o3HipGetDeviceProperties)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    names = _declared()
    for required in ("fe2o3HipGetDeviceProperties", "fe2o3_tiled_gemm_lds_slice1_v1",
                     "fe2o3_tiled_gemm_general_v1", "fe2o3_scalar_gemm_v1", "fe2o3_gemm_bf16_nt",
                     "fe2o3_row_softmax_v1", "fe2o3_flash_attention_fwd",
                     "fe2o3_moe_top2_route_f32_t8_e4_k2_c4_v1", "fe2o3_moe_ffn_top2",
                     "fe2o3_gemm_fp8_nt"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from fe2o3_amd import _lib
    L = C.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(L, n)]
    assert missing == []


def test_ctypes_table_matches_header():
    from fe2o3_amd import _lib
    assert sorted(_lib.SIGNATURES) == _declared()


def test_property_record_layout():
    from fe2o3_amd._lib import Fe2o3HipDeviceProperties as P
    assert C.sizeof(P) == 312 and C.alignment(P) == 8
    offsets = {"gcn_arch_name": 0, "warp_size": 256, "max_threads_per_block": 260,
               "max_block_dim": 264, "max_grid_dim": 276, "shared_mem_per_block": 288,
               "shared_mem_per_block_optin": 296, "architecture_features": 304}
    for name, off in offsets.items():
        assert getattr(P, name).offset == off


# Host-side validation runs before any HIP call, so these need no GPU.
def test_length_and_shape_validation_without_gpu():
    from fe2o3_amd import _lib
    L = _lib.lib()
    assert L.fe2o3_tiled_gemm_lds_slice1_v1(None, 255, None, 256, None, 256, None) == -2
    assert L.fe2o3_tiled_gemm_general_v1(None, 0, None, 0, None, 0, 4, 4, 4, 3, 4, 4, 1.0, 0.0,
                                         None) == -4
    assert L.fe2o3_gemm_bf16_nt(None, 10, None, 10, None, 10, 4, 4, 4, None) == -2
    assert L.fe2o3_row_softmax(None, 0, None, 0, None, 0, 4, 0, None) == -3
    assert L.fe2o3_flash_attention_fwd(None, 0, None, 0, None, 0, None, 0, None, 0, 1, 1, 128, 64,
                                       0, 0.1, None) == -3
    # one head's K/V must fit the kernel's 32-bit buffer range (seq * 256 B < 2^31)
    big = (1 << 23) * 128
    assert L.fe2o3_flash_attention_fwd(None, big, None, big, None, big, None, big, None, 0, 1, 1,
                                       1 << 23, 128, 0, 0.1, None) == -3
    ok = ((1 << 23) - 128) * 128  # largest seq that fits passes the shape checks
    assert L.fe2o3_flash_attention_fwd(None, ok, None, ok, None, ok, None, ok, None, 0, 1, 1,
                                       (1 << 23) - 128, 128, 0, 0.1, None) == -19
    assert L.fe2o3_moe_top2_route(None, 0, 0, None, 0, None, 0, None, 0, None, 0, None, 0, None,
                                  0, None, 0, None, 0, 0, 1, 0, None) == -3
    # any m, n, k is a valid shape; the null operands are refused before a launch
    assert L.fe2o3_gemm_fp8_nt(None, 256 * 100, None, 256 * 100, None, None, None, 256 * 256,
                               256, 256, 100, None) == -19
    assert L.fe2o3_gemm_fp8_nt(None, 0, None, 0, None, None, None, 0, 0, 0, 0, None) == 0
    assert L.fe2o3_moe_ffn_workspace_bytes(4096, 4096, 14336, 8) >= 8192 * (4096 * 6 + 14336 * 2)
    assert b"length" in L.fe2o3_status_string(-2)


def test_kernel_resource_record_and_registry_without_gpu():
    """The record layout, and the per-entry kernel counts: the lookup needs
    no GPU; only the resource query itself does."""
    import ctypes
    from fe2o3_amd import _lib
    R = _lib.Fe2o3KernelResources
    assert ctypes.sizeof(R) == 120
    offsets = {"kernel": 0, "workgroup_size": 96, "static_lds_bytes": 100,
               "dynamic_lds_bytes": 104, "private_segment_bytes": 108, "vgprs": 112,
               "max_threads_per_workgroup": 116}
    for name, off in offsets.items():
        assert getattr(R, name).offset == off
    L = _lib.lib()
    expected = {"fe2o3_gemm_bf16_nt": 24, "fe2o3_flash_attention_fwd": 4, "fe2o3_moe_ffn_top2": 5,
                "fe2o3_gemm_fp8_nt": 24, "fe2o3_row_softmax": 13, "fe2o3_moe_routing_check": 7,
                "fe2o3_wave64_collectives_v1": 1, "fe2o3_fp8_fnuz_from_f32": 4,
                "fe2o3_fp8_fnuz_to_f32": 4, "fe2o3_tiled_gemm_general_v1": 12,
                "fe2o3_bf16_from_f32": 2, "no_such_entry": 0}
    for entry, n in expected.items():
        count = ctypes.c_uint32(12345)
        assert L.fe2o3_kernel_resources(entry.encode(), 10**6, None, ctypes.byref(count)) == -2
        assert count.value == n, entry
    # every declared kernel entry point (not the runtime seam, and not the
    # code-object lifecycles, whose kernels live in their own loaded modules)
    # registers a kernel
    kernel_entries = [n for n in _declared()
                      if not n.startswith(("fe2o3_rt_", "fe2o3Hip", "fe2o3_lds_gemm_slice1_",
                                           "fe2o3_protected_"))
                      and n not in ("fe2o3_status_string", "fe2o3_kernel_resources",
                                    "fe2o3_moe_ffn_workspace_bytes", "fe2o3_sha256_v1")]
    for entry in kernel_entries:
        count = ctypes.c_uint32(0)
        L.fe2o3_kernel_resources(entry.encode(), 10**6, None, ctypes.byref(count))
        assert count.value >= 1, entry


def test_fault_point_fails_closed(monkeypatch):
    """FE2O3_FAULT_POINT forces an entry point to fail before any launch."""
    from fe2o3_amd import _lib
    monkeypatch.setenv("FE2O3_FAULT_POINT", "fe2o3_gemm_bf16_nt")
    L = _lib.lib()
    assert L.fe2o3_gemm_bf16_nt(None, 0, None, 0, None, 0, 0, 0, 0, None) == -23


def test_typed_prepare_rejects_wrong_element_type():
    from fe2o3_amd import kernels
    from fe2o3_amd.runtime import DeviceBuffer
    import numpy as np
    fake = DeviceBuffer.__new__(DeviceBuffer)
    fake.dtype, fake.count, fake.ptr, fake.nbytes = np.dtype(np.float32), 256, None, 1024
    k = kernels.tiled_gemm_lds_slice1_gpu.Kernel(ctx=None)
    with pytest.raises(TypeError):
        k.prepare(fake, fake, fake)
    fake.ptr = None


def test_tiled_gemm_v1_plan_without_gpu():
    """examples/tiled_gemm_v1's plan_v1 outcomes that launch nothing, through
    the C-ABI entry point (validation runs before any HIP call): every
    EDGE_CASES_V1 row that plans no dispatch or a rejection, the extreme
    empty shapes (no operand buffers), the A/B/C byte-overflow order, wrong
    lengths, and empty outputs that name operand buffers."""
    from golden import reference_vectors as rv
    from fe2o3_amd import _lib
    L = _lib.lib()
    code = {"m-tail": -24, "n-tail": -25, "k-tail": -26, "no-dispatch": 0}
    seen = set()
    for name, m, n, k, outcome in rv.EDGE_CASES_V1:
        if outcome not in code:
            continue
        empty = m == 0 or n == 0
        la, lb, lc = (0, 0, 0) if empty else (m * k, k * n, m * n)
        assert L.fe2o3_tiled_gemm_v1(None, la, None, lb, None, lc, m, n, k, None) == code[outcome], name
        seen.add(outcome)
    assert seen == set(code)
    for m, n, k in rv.EXTREME_EMPTY_V1:
        assert L.fe2o3_tiled_gemm_v1(None, 0, None, 0, None, 0, m, n, k, None) == 0
        # an empty output requires zero-length operands
        assert L.fe2o3_tiled_gemm_v1(None, 1, None, 0, None, 0, m, n, k, None) == -2
    for m, n, k, _ in rv.BYTE_OVERFLOW_V1:
        assert L.fe2o3_tiled_gemm_v1(None, 0, None, 0, None, 0, m, n, k, None) == -16
    assert L.fe2o3_tiled_gemm_v1(None, 255, None, 256, None, 256, 16, 16, 16, None) == -2
    # a tail is reported after the lengths are checked, M before N before K
    assert L.fe2o3_tiled_gemm_v1(None, 17 * 15, None, 15 * 31, None, 17 * 31, 17, 31, 15,
                                 None) == -24
    assert L.fe2o3_tiled_gemm_v1(None, 16 * 15, None, 15 * 31, None, 16 * 31, 16, 31, 15,
                                 None) == -25
    # K = 0 with tails in M or N still rejects; K = 0 itself is a host fill
    assert L.fe2o3_tiled_gemm_v1(None, 0, None, 0, None, 17 * 16, 17, 16, 0, None) == -24
    assert b"16-row tile" in L.fe2o3_status_string(-24)


SLICE1_RECORDS = ["Fe2o3Slice1ErrorV1", "Fe2o3Slice1BufferContractV1", "Fe2o3Slice1ContractV1",
                  "Fe2o3Slice1InspectionV1", "Fe2o3Slice1ArtifactV1", "Fe2o3Slice1JoinFactsV1",
                  "Fe2o3Slice1GeometryV1", "Fe2o3Slice1EnvironmentV1", "Fe2o3Slice1LoadV1",
                  "Fe2o3Slice1ResolutionV1", "Fe2o3Slice1ResourcesV1", "Fe2o3Slice1ImplicitV1",
                  "Fe2o3Slice1DispatchV1", "Fe2o3Slice1UnloadV1", "Fe2o3Slice1AdapterV1",
                  "Fe2o3Slice1ReceiptV1", "Fe2o3Slice1ObservationV1"]


def test_lifecycle_record_layouts_match_the_header(tmp_path):
    """Every lifecycle record's size, alignment and field offsets as the C
    compiler lays them out from include/fe2o3_mi355x.h equal the ctypes
    mirror's."""
    import shutil
    import subprocess
    from fe2o3_amd import _lib
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "fe2o3_mi355x.h"',
             "int main(void) {"]
    expect = []
    for name in SLICE1_RECORDS:
        rec = getattr(_lib, name)
        lines.append(f'printf("%zu %zu\\n", sizeof({name}), _Alignof({name}));')
        expect.append(f"{C.sizeof(rec)} {C.alignment(rec)}")
        for field, _ in rec._fields_:
            lines.append(f'printf("%zu\\n", offsetof({name}, {field}));')
            expect.append(str(getattr(rec, field).offset))
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([cc, "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    assert got[:-1] == expect


def test_module_seam_refuses_null_arguments_without_gpu():
    """lib.rs:144-165's module subset: every NULL out-pointer, name, image or
    handle is refused with FE2O3_ERR_NULL (-19) before HIP is called."""
    from fe2o3_amd import _lib
    L = _lib.lib()
    null = -19
    mod = C.c_void_p(0x1234)
    fn = C.c_void_p(0x5678)
    assert L.fe2o3_rt_module_load(None, b"x.co") == null
    assert L.fe2o3_rt_module_load(C.byref(mod), None) == null
    assert L.fe2o3_rt_module_load_data(None, C.c_void_p(1)) == null
    assert L.fe2o3_rt_module_load_data(C.byref(mod), None) == null
    assert L.fe2o3_rt_module_unload(None) == null
    assert L.fe2o3_rt_module_get_function(None, C.c_void_p(1), b"k") == null
    assert L.fe2o3_rt_module_get_function(C.byref(fn), None, b"k") == null
    assert L.fe2o3_rt_module_get_function(C.byref(fn), C.c_void_p(1), None) == null
    assert L.fe2o3_rt_module_launch_kernel(None, 1, 1, 1, 64, 1, 1, 0, None, None, None) == null
    assert L.fe2o3_status_string(null) == b"required pointer is NULL"


def test_published_code_object_is_the_embedded_one():
    """The build places the slice-1 code object next to the library for the
    module entry points; its SHA-256 is the lifecycle artifact's finalizer
    identity, i.e. the bytes the library embeds."""
    import hashlib
    from fe2o3_amd import _lib, lifecycle
    path = os.path.join(os.path.dirname(_lib.LIB_PATH), "tiled_gemm_lds_v1.co")
    with open(path, "rb") as f:
        data = f.read()
    assert hashlib.sha256(data).digest() == bytes(lifecycle.artifact().finalizer_identity)
