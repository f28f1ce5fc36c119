"""Kernel resource observation on the GPU (fe2o3_kernel_resources): every
kernel behind every entry point runs without scratch (private segment 0:
no register spills), fits the CU's 160 KiB of LDS with its launch's dynamic
request, and launches within its workgroup limit.  The reference rejects a
loaded kernel whose observed group/private segments drift from the expected
ones (crates/fe2o3-host/src/generated_lds_gemm_lifecycle.rs:883-900); here
the expected values are the hot kernels' design figures."""
from __future__ import annotations

import pytest

from test_abi import _declared

pytestmark = pytest.mark.gpu

LDS_PER_CU = 160 * 1024


def _entries():
    return [n for n in _declared() if not n.startswith(("fe2o3_rt_", "fe2o3Hip"))
            and n not in ("fe2o3_status_string", "fe2o3_kernel_resources",
                          "fe2o3_moe_ffn_workspace_bytes")]


def test_every_kernel_is_spill_free_and_fits(gpu):
    from fe2o3_amd import kernels
    seen = 0
    for entry in _entries():
        for r in kernels.kernel_resources(entry):
            seen += 1
            assert r["private_segment_bytes"] == 0, (entry, r)
            assert r["static_lds_bytes"] + r["dynamic_lds_bytes"] <= LDS_PER_CU, (entry, r)
            assert 0 < r["workgroup_size"] <= r["max_threads_per_workgroup"], (entry, r)
    assert seen >= 40


@pytest.mark.parametrize("entry,kernel,dynamic_lds,threads", [
    ("fe2o3_gemm_bf16_nt", "gemm_bf16_nt_256_kernel", 128 * 1024, 256),
    ("fe2o3_gemm_bf16_nt", "gemm_bf16_nt_256_kernel<staged>", 128 * 1024, 256),
    ("fe2o3_gemm_fp8_nt", "gemm_fp8_kernel", 128 * 1024, 256),
    ("fe2o3_gemm_fp8_nt", "gemm_fp8_kernel<staged>", 128 * 1024, 256),
    ("fe2o3_flash_attention_fwd", "flash_fwd_kernel<false>", 64 * 1024, 256),
    ("fe2o3_flash_attention_fwd", "flash_fwd_kernel<true>", 64 * 1024, 256),
    ("fe2o3_moe_ffn_top2", "gate_up_kernel", 136 * 1024, 256),
    ("fe2o3_moe_ffn_top2", "gate_up_kernel<gathered>", 136 * 1024, 256),
    ("fe2o3_moe_ffn_top2", "down_kernel", 136 * 1024, 256),
    ("fe2o3_moe_routing_check", "routing_check_kernel", 96 * 1024, 128)])
def test_hot_kernels_match_design(gpu, entry, kernel, dynamic_lds, threads):
    from fe2o3_amd import kernels
    rows = {r["kernel"]: r for r in kernels.kernel_resources(entry)}
    r = rows[kernel]
    assert r["dynamic_lds_bytes"] == dynamic_lds
    assert r["private_segment_bytes"] == 0
    assert r["workgroup_size"] == threads
