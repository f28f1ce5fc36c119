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
