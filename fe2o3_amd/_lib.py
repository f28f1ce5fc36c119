"""ctypes binding of libfe2o3_mi355x.so (the C-ABI of include/fe2o3_mi355x.h).

Loading fails loudly: there is no CPU fallback anywhere in this package.  If
the shared library has not been built (``python -c "import __graft_entry__ as
g; g.build()"`` or ``make -C fe2o3_amd/csrc``) every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfe2o3_mi355x.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "fe2o3_mi355x.h")

_lib = None

i32, u32, u64, f32, sz = C.c_int32, C.c_uint32, C.c_uint64, C.c_float, C.c_size_t
vp = C.c_void_p
pvp = C.POINTER(C.c_void_p)
pi32 = C.POINTER(C.c_int32)
pf32 = C.POINTER(C.c_float)


class Fe2o3HipDeviceProperties(C.Structure):
    """crates/fe2o3-hip-sys/src/lib.rs:49-60 (312 bytes, 8-aligned)."""

    _fields_ = [
        ("gcn_arch_name", C.c_char * 256),
        ("warp_size", C.c_int32),
        ("max_threads_per_block", C.c_int32),
        ("max_block_dim", C.c_int32 * 3),
        ("max_grid_dim", C.c_int32 * 3),
        ("shared_mem_per_block", C.c_uint64),
        ("shared_mem_per_block_optin", C.c_uint64),
        ("architecture_features", C.c_uint64),
    ]


class Fe2o3KernelResources(C.Structure):
    """Resource record of one kernel behind an entry point (120 bytes)."""

    _fields_ = [
        ("kernel", C.c_char * 96),
        ("workgroup_size", C.c_uint32),
        ("static_lds_bytes", C.c_uint32),
        ("dynamic_lds_bytes", C.c_uint32),
        ("private_segment_bytes", C.c_uint32),
        ("vgprs", C.c_uint32),
        ("max_threads_per_workgroup", C.c_uint32),
    ]


# ---- exact LDS GEMM lifecycle records (fe2o3_lds_gemm_slice1_*) ----------------------

u8, c_char = C.c_uint8, C.c_char


class Fe2o3Slice1ErrorV1(C.Structure):
    _fields_ = [("kind", i32), ("index", i32), ("adapter_status", i32), ("reserved", i32),
                ("expected", u64), ("actual", u64), ("field", c_char * 64)]


class Fe2o3Slice1BufferContractV1(C.Structure):
    _fields_ = [("role", u32), ("element", u32), ("elements", u64), ("bytes", u64),
                ("length_identity", u8 * 32), ("ownership", u32), ("access", u32),
                ("alias", u32), ("reserved", u32)]


class Fe2o3Slice1ContractV1(C.Structure):
    _fields_ = [("profile", u32), ("code_object_version", u32), ("target", c_char * 32),
                ("identity", u8 * 32), ("grid", u32 * 3), ("workgroup", u32 * 3),
                ("wavefront_size", u32), ("explicit_kernarg_bytes", u32),
                ("complete_kernarg_bytes", u32), ("kernarg_alignment", u32),
                ("static_lds_bytes", u32), ("lds_allocations", u32),
                ("lds_bytes_per_allocation", u32), ("lds_alignment", u32),
                ("buffers", Fe2o3Slice1BufferContractV1 * 3)]


class Fe2o3Slice1InspectionV1(C.Structure):
    _fields_ = [("byte_len", u64), ("code_object_version", u32), ("e_flags", u32),
                ("target", c_char * 64), ("kd_group_segment_bytes", u32),
                ("kd_private_segment_bytes", u32), ("kd_kernarg_bytes", u32),
                ("kd_wavefront_size", u32), ("md_kernarg_bytes", u32),
                ("md_kernarg_alignment", u32), ("md_group_segment_bytes", u32),
                ("md_private_segment_bytes", u32), ("md_wavefront_size", u32),
                ("md_max_flat_workgroup_size", u32), ("explicit_args", u32),
                ("explicit_bytes", u32), ("implicit_offset", u32), ("implicit_bytes", u32),
                ("sgpr_spills", u32), ("vgpr_spills", u32), ("uses_dynamic_stack", u32),
                ("reserved", u32)]


class Fe2o3Slice1ArtifactV1(C.Structure):
    _fields_ = [("finalizer_identity", u8 * 32), ("build_digest", u8 * 32),
                ("import_identity", u8 * 32), ("profile_identity", u8 * 32),
                ("contract", Fe2o3Slice1ContractV1), ("inspection", Fe2o3Slice1InspectionV1)]


class Fe2o3Slice1JoinFactsV1(C.Structure):
    _fields_ = [("import_matches", u8), ("profile_matches", u8), ("contract_matches", u8),
                ("finalized_output_matches", u8), ("inspection_matches", u8),
                ("host_profile_identity_matches", u8), ("reserved", u8 * 2),
                ("contract", Fe2o3Slice1ContractV1), ("host_target", c_char * 32),
                ("host_profile", u32), ("host_grid", u32 * 3), ("host_workgroup", u32 * 3),
                ("host_static_lds", u32), ("host_dynamic_lds", u32),
                ("host_explicit_kernarg", u32), ("host_complete_kernarg", u32),
                ("host_kernarg_alignment", u32), ("host_length_identities", (u8 * 32) * 3)]


class Fe2o3Slice1GeometryV1(C.Structure):
    _fields_ = [("grid", u32 * 3), ("workgroup", u32 * 3), ("dynamic_lds_bytes", u32)]


class Fe2o3Slice1EnvironmentV1(C.Structure):
    _fields_ = [("runtime_instance", u8 * 16), ("physical_target", c_char * 64),
                ("hip_ordinal", i32), ("physical_uuid", u8 * 16), ("agent_target", c_char * 64),
                ("agent_handle", u64), ("agent_runtime_instance", u8 * 16),
                ("agent_physical_uuid", u8 * 16)]


class Fe2o3Slice1LoadV1(C.Structure):
    _fields_ = [("digest", u8 * 32), ("byte_len", u64), ("runtime_instance", u8 * 16),
                ("agent_handle", u64), ("executable_object", u8 * 16)]


class Fe2o3Slice1ResolutionV1(C.Structure):
    _fields_ = [("executable_object", u8 * 16), ("kernel_object", u8 * 16),
                ("symbol", c_char * 64), ("kernarg_segment_bytes", u64),
                ("kernarg_alignment", u64)]


class Fe2o3Slice1ResourcesV1(C.Structure):
    _fields_ = [("executable_object", u8 * 16), ("kernel_object", u8 * 16),
                ("group_segment_bytes", u32), ("private_segment_bytes", u32)]


class Fe2o3Slice1ImplicitV1(C.Structure):
    _fields_ = [("executable_object", u8 * 16), ("kernel_object", u8 * 16),
                ("geometry", Fe2o3Slice1GeometryV1), ("explicit_bytes", u64),
                ("implicit_offset", u64), ("implicit_bytes", u64), ("completed", u32),
                ("reserved", u32)]


class Fe2o3Slice1DispatchV1(C.Structure):
    _fields_ = [("dispatch_identity", u8 * 16), ("executable_object", u8 * 16),
                ("kernel_object", u8 * 16), ("geometry", Fe2o3Slice1GeometryV1),
                ("completed", u32)]


class Fe2o3Slice1UnloadV1(C.Structure):
    _fields_ = [("executable_object", u8 * 16), ("runtime_instance", u8 * 16),
                ("agent_handle", u64), ("released", u32), ("reserved", u32)]


pu64 = C.POINTER(u64)
SLICE1_CONTEXT_FN = C.CFUNCTYPE(i32, vp, C.POINTER(u8 * 16))
SLICE1_ENVIRONMENT_FN = C.CFUNCTYPE(i32, vp, C.POINTER(Fe2o3Slice1EnvironmentV1))
SLICE1_LOAD_FN = C.CFUNCTYPE(i32, vp, C.POINTER(u8), u64, C.POINTER(u8 * 32), pu64,
                             C.POINTER(Fe2o3Slice1LoadV1))
SLICE1_RESOLVE_FN = C.CFUNCTYPE(i32, vp, u64, C.c_char_p, pu64, C.POINTER(Fe2o3Slice1ResolutionV1))
SLICE1_RESOURCES_FN = C.CFUNCTYPE(i32, vp, u64, u64, C.POINTER(Fe2o3Slice1ResourcesV1))
SLICE1_IMPLICIT_FN = C.CFUNCTYPE(i32, vp, u64, u64, C.POINTER(Fe2o3Slice1GeometryV1), u64, u64, u64,
                                 C.POINTER(u8), u64, C.POINTER(Fe2o3Slice1ImplicitV1))
SLICE1_LAUNCH_FN = C.CFUNCTYPE(i32, vp, u64, u64, C.POINTER(Fe2o3Slice1GeometryV1), C.POINTER(u8),
                               u64, C.POINTER(Fe2o3Slice1DispatchV1))
SLICE1_DROP_KERNEL_FN = C.CFUNCTYPE(None, vp, u64)
SLICE1_UNLOAD_FN = C.CFUNCTYPE(i32, vp, u64, C.POINTER(Fe2o3Slice1UnloadV1))
SLICE1_DROP_ADAPTER_FN = C.CFUNCTYPE(None, vp)
SLICE1_RELEASE_FN = C.CFUNCTYPE(None, vp)


class Fe2o3Slice1AdapterV1(C.Structure):
    _fields_ = [("self", vp), ("context_identity", SLICE1_CONTEXT_FN),
                ("observe_environment", SLICE1_ENVIRONMENT_FN),
                ("load_executable", SLICE1_LOAD_FN), ("resolve_kernel", SLICE1_RESOLVE_FN),
                ("observe_resources", SLICE1_RESOURCES_FN),
                ("initialize_implicit_kernarg", SLICE1_IMPLICIT_FN),
                ("launch_and_wait", SLICE1_LAUNCH_FN), ("drop_kernel", SLICE1_DROP_KERNEL_FN),
                ("unload_executable", SLICE1_UNLOAD_FN), ("drop_adapter", SLICE1_DROP_ADAPTER_FN)]


class Fe2o3Slice1ReceiptV1(C.Structure):
    _fields_ = [("finalizer_identity", u8 * 32), ("import_identity", u8 * 32),
                ("profile_identity", u8 * 32), ("executable_object", u8 * 16),
                ("kernel_object", u8 * 16), ("dispatch_identity", u8 * 16),
                ("unload_identity", u8 * 32)]


class Fe2o3Slice1ObservationV1(C.Structure):
    _fields_ = [("state", i32), ("leases_retained", u32), ("holds_executable", u32),
                ("holds_kernel", u32), ("environment", Fe2o3Slice1EnvironmentV1),
                ("load", Fe2o3Slice1LoadV1), ("resolution", Fe2o3Slice1ResolutionV1),
                ("resources", Fe2o3Slice1ResourcesV1), ("dispatch_identity", u8 * 16),
                ("last_error", Fe2o3Slice1ErrorV1)]

# ---- protected profile lifecycles (fe2o3_protected_*) ----------------------------------

PROTECTED_MAX_REGIONS = 8


class Fe2o3ProtectedRegionV1(C.Structure):
    _fields_ = [("address", vp), ("elements", u64)]


class Fe2o3ProtectedProfileV1(C.Structure):
    _fields_ = [("profile", u32), ("code_object_version", u32), ("name", C.c_char * 32),
                ("target", C.c_char * 32), ("symbol", C.c_char * 64), ("grid", u32 * 3),
                ("workgroup", u32 * 3), ("dynamic_lds_bytes", u32), ("static_lds_bytes", u32),
                ("private_segment_bytes", u32), ("explicit_kernarg_bytes", u32),
                ("complete_kernarg_bytes", u32), ("kernarg_alignment", u32),
                ("hsa_kernarg_alignment", u32), ("regions", u32),
                ("region_elements", u64 * PROTECTED_MAX_REGIONS),
                ("region_element_bytes", u32 * PROTECTED_MAX_REGIONS),
                ("region_writes", u32 * PROTECTED_MAX_REGIONS), ("shape", u32 * 4),
                ("receipt_fields", u32), ("host_fields", u32),
                ("receipt_field", (C.c_char * 40) * 16), ("host_field", (C.c_char * 40) * 16)]


class Fe2o3ProtectedArtifactV1(C.Structure):
    _fields_ = [("identity", u8 * 32), ("profile_identity", u8 * 32),
                ("artifact_identity", u8 * 32), ("build_digest", u8 * 32),
                ("source_digest", u8 * 32), ("compiler_identity", u8 * 32),
                ("inspection", Fe2o3Slice1InspectionV1), ("profile", Fe2o3ProtectedProfileV1)]


class Fe2o3ProtectedJoinFactsV1(C.Structure):
    _fields_ = [("profile", u32), ("receipt", u8 * 16), ("host_target", C.c_char * 32),
                ("host_shape", u32 * 4), ("host_argument_elements", u64),
                ("host_grid", u32 * 3), ("host_workgroup", u32 * 3),
                ("host_code_object_version", u32), ("host_explicit_kernarg", u32),
                ("host_complete_kernarg", u32), ("host_kernarg_alignment", u32),
                ("host_policy", u32)]


class Fe2o3ProtectedReceiptV1(C.Structure):
    _fields_ = [("identity", u8 * 32), ("artifact_identity", u8 * 32),
                ("executable_object", u8 * 16), ("kernel_object", u8 * 16),
                ("dispatch_identity", u8 * 16), ("unload_identity", u8 * 32)]


# name -> (restype, argtypes).  Order and meaning follow the header.
SIGNATURES = {
    "fe2o3_status_string": (C.c_char_p, [i32]),
    "fe2o3HipGetDeviceProperties": (i32, [i32, C.POINTER(Fe2o3HipDeviceProperties)]),
    "fe2o3_rt_init": (i32, [u32]),
    "fe2o3_rt_get_device_count": (i32, [pi32]),
    "fe2o3_rt_set_device": (i32, [i32]),
    "fe2o3_rt_get_device": (i32, [pi32]),
    "fe2o3_rt_device_rates": (i32, [i32, pi32, pi32, pi32, pi32]),
    "fe2o3_rt_require_gfx950": (i32, [i32]),
    "fe2o3_rt_device_synchronize": (i32, []),
    "fe2o3_rt_stream_create": (i32, [pvp]),
    "fe2o3_rt_stream_destroy": (i32, [vp]),
    "fe2o3_rt_stream_synchronize": (i32, [vp]),
    "fe2o3_rt_event_create": (i32, [pvp, u32]),
    "fe2o3_rt_event_destroy": (i32, [vp]),
    "fe2o3_rt_event_record": (i32, [vp, vp]),
    "fe2o3_rt_event_synchronize": (i32, [vp]),
    "fe2o3_rt_event_query": (i32, [vp]),
    "fe2o3_rt_event_elapsed_ms": (i32, [pf32, vp, vp]),
    "fe2o3_rt_malloc": (i32, [pvp, sz]),
    "fe2o3_rt_free": (i32, [vp]),
    "fe2o3_rt_host_malloc": (i32, [pvp, sz]),
    "fe2o3_rt_host_free": (i32, [vp]),
    "fe2o3_rt_memcpy_async": (i32, [vp, vp, sz, u32, vp]),
    "fe2o3_rt_memcpy": (i32, [vp, vp, sz, u32]),
    "fe2o3_rt_memset_async": (i32, [vp, i32, sz, vp]),
    "fe2o3_rt_module_load": (i32, [C.POINTER(vp), C.c_char_p]),
    "fe2o3_rt_module_load_data": (i32, [C.POINTER(vp), vp]),
    "fe2o3_rt_module_unload": (i32, [vp]),
    "fe2o3_rt_module_get_function": (i32, [C.POINTER(vp), vp, C.c_char_p]),
    "fe2o3_rt_module_launch_kernel": (i32, [vp, u32, u32, u32, u32, u32, u32, u32, vp,
                                            C.POINTER(vp), C.POINTER(vp)]),
    "fe2o3_fill_normal_bf16": (i32, [vp, u64, u64, u64, f32, u64, vp]),
    "fe2o3_fill_normal_f32": (i32, [vp, u64, u64, u64, f32, u64, vp]),
    "fe2o3_fill_uniform_f32": (i32, [vp, u64, u64, u64, u64, vp]),
    "fe2o3_tiled_gemm_lds_slice1_v1": (i32, [vp, u64, vp, u64, vp, u64, vp]),
    "fe2o3_tiled_gemm_v1": (i32, [vp, u64, vp, u64, vp, u64, u32, u32, u32, vp]),
    "fe2o3_tiled_gemm_general_v1": (
        i32, [vp, u64, vp, u64, vp, u64, u32, u32, u32, u32, u32, u32, f32, f32, vp]),
    "fe2o3_tiled_gemm_general_vector_a_v1": (
        i32, [vp, u64, vp, u64, vp, u64, u32, u32, u32, u32, u32, u32, f32, f32, vp]),
    "fe2o3_scalar_gemm_v1": (i32, [vp, u64, vp, u64, vp, u64, u32, u32, u32, vp]),
    "fe2o3_gemm_bf16_nt": (i32, [vp, u64, vp, u64, vp, u64, u32, u32, u32, vp]),
    "fe2o3_row_softmax_v1": (i32, [vp, u64, vp, u64, vp]),
    "fe2o3_row_softmax": (i32, [vp, u64, vp, u64, vp, u64, u64, u64, vp]),
    "fe2o3_flash_attention_causal_f32_b1_h1_n8_d16_v1": (
        i32, [vp, u64, vp, u64, vp, u64, vp, u64, vp]),
    "fe2o3_flash_attention_fwd": (
        i32, [vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, u32, u32, u32, u32, i32, f32, vp]),
    "fe2o3_moe_top2_route_f32_t8_e4_k2_c4_v1": (
        i32, [vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp]),
    "fe2o3_moe_top2_route": (
        i32, [vp, u64, u32, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64,
              vp, u64, u32, u32, u32, vp]),
    "fe2o3_moe_expert_gemm_bf16_m16_n16_k16_v1": (i32, [vp, u64, vp, u64, vp, u64, vp]),
    "fe2o3_moe_expert_combine_f32_t8_k2_o16_v1": (
        i32, [vp, u64, vp, u64, vp, u64, vp, u64, vp]),
    "fe2o3_moe_ffn_workspace_bytes": (u64, [u32, u32, u32, u32]),
    "fe2o3_moe_ffn_top2": (
        i32, [vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64,
              vp, u64, vp, u64, u32, u32, u32, u32, vp]),
    "fe2o3_moe_ffn_top2_noalloc": (
        i32, [vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64,
              vp, u64, u32, u32, u32, u32, vp]),
    "fe2o3_amax_f32": (i32, [vp, u64, vp, vp]),
    "fe2o3_fp8_scale_from_amax": (i32, [vp, vp, vp]),
    "fe2o3_quantize_e4m3": (i32, [vp, u64, vp, vp, u64, vp]),
    "fe2o3_fp8_fnuz_from_f32": (i32, [vp, u64, vp, u64, i32, vp]),
    "fe2o3_fp8_fnuz_to_f32": (i32, [vp, u64, vp, u64, i32, vp]),
    "fe2o3_bf16_from_f32": (i32, [vp, u64, vp, u64, vp]),
    "fe2o3_gemm_fp8_nt": (i32, [vp, u64, vp, u64, vp, vp, vp, u64, u32, u32, u32, vp]),
    "fe2o3_moe_routing_check": (
        i32, [vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, u32, u32, u32, vp,
              u64, vp]),
    "fe2o3_kernel_resources": (
        i32, [C.c_char_p, u32, C.POINTER(Fe2o3KernelResources), C.POINTER(u32)]),
    "fe2o3_wave64_collectives_v1": (i32, [vp, u64, u64, vp, u64, vp, u64, vp, u64, vp]),
    "fe2o3_wave64_collectives_rows": (
        i32, [vp, u64, vp, u64, vp, u64, vp, u64, vp, u64, u64, vp]),
    "fe2o3_lds_reduce_i32_v1": (i32, [vp, u64, vp, u64, vp]),
    "fe2o3_scoped_atomic_add_u32_v1": (i32, [vp, u64, vp, u64, vp, vp]),
    "fe2o3_sha256_v1": (i32, [vp, u64, C.POINTER(u8 * 32)]),
    "fe2o3_lds_gemm_slice1_artifact_v1": (i32, [C.POINTER(Fe2o3Slice1ArtifactV1)]),
    "fe2o3_lds_gemm_slice1_join_facts_v1": (i32, [C.POINTER(Fe2o3Slice1JoinFactsV1)]),
    "fe2o3_lds_gemm_slice1_validate_join_v1": (
        i32, [C.POINTER(Fe2o3Slice1JoinFactsV1), C.POINTER(Fe2o3Slice1ErrorV1)]),
    "fe2o3_lds_gemm_slice1_join_v1": (
        i32, [vp, u64, vp, u64, vp, u64, i32, SLICE1_RELEASE_FN, vp, pvp,
              C.POINTER(Fe2o3Slice1ErrorV1)]),
    "fe2o3_lds_gemm_slice1_hip_adapter_v1": (i32, [i32, C.POINTER(Fe2o3Slice1AdapterV1)]),
    "fe2o3_lds_gemm_slice1_context_identity_v1": (i32, [i32, C.POINTER(u8 * 16)]),
    "fe2o3_lds_gemm_slice1_load_v1": (
        i32, [vp, C.POINTER(Fe2o3Slice1AdapterV1), C.POINTER(Fe2o3Slice1ErrorV1)]),
    "fe2o3_lds_gemm_slice1_dispatch_and_wait_v1": (i32, [vp, C.POINTER(Fe2o3Slice1ErrorV1)]),
    "fe2o3_lds_gemm_slice1_unload_v1": (i32, [vp, C.POINTER(Fe2o3Slice1ReceiptV1)]),
    "fe2o3_lds_gemm_slice1_release_v1": (None, [vp]),
    "fe2o3_lds_gemm_slice1_observe_v1": (i32, [vp, C.POINTER(Fe2o3Slice1ObservationV1)]),
    "fe2o3_protected_profile_v1": (i32, [u32, C.POINTER(Fe2o3ProtectedProfileV1)]),
    "fe2o3_protected_artifact_v1": (i32, [u32, C.POINTER(Fe2o3ProtectedArtifactV1)]),
    "fe2o3_protected_join_facts_v1": (i32, [u32, C.POINTER(Fe2o3ProtectedJoinFactsV1)]),
    "fe2o3_protected_validate_join_v1": (
        i32, [C.POINTER(Fe2o3ProtectedJoinFactsV1), C.POINTER(Fe2o3Slice1ErrorV1)]),
    "fe2o3_protected_join_v1": (
        i32, [u32, C.POINTER(Fe2o3ProtectedRegionV1), u32, i32, SLICE1_RELEASE_FN, vp, pvp,
              C.POINTER(Fe2o3Slice1ErrorV1)]),
    "fe2o3_protected_load_v1": (
        i32, [vp, C.POINTER(Fe2o3Slice1AdapterV1), C.POINTER(Fe2o3Slice1ErrorV1)]),
    "fe2o3_protected_dispatch_and_wait_v1": (i32, [vp, C.POINTER(Fe2o3Slice1ErrorV1)]),
    "fe2o3_protected_unload_v1": (i32, [vp, C.POINTER(Fe2o3ProtectedReceiptV1)]),
    "fe2o3_protected_release_v1": (None, [vp]),
    "fe2o3_protected_observe_v1": (i32, [vp, C.POINTER(Fe2o3Slice1ObservationV1)]),
}


class LibraryMissing(ImportError):
    pass


def lib():
    """The loaded library with every signature declared.  Raises
    LibraryMissing when the .so has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is not built; run __graft_entry__.build() "
                "(no CPU fallback exists)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name, None)
            if fn is None:  # reported by tests/test_abi.py; calling it raises AttributeError
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def status_string(status: int) -> str:
    s = lib().fe2o3_status_string(status)
    return s.decode() if s else f"status {status}"
