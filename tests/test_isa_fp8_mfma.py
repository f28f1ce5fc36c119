"""The fp8 GEMM tiles (gemm_pipe::Fp8Mma16, both tile forms) call the
scaled f8f6f4 MFMA builtin with both scale operands 0, for which the
compiler selects the unscaled v_mfma_f32_16x16x128_f8f6f4: one instruction
per MFMA, with no v_mfma_ld_scale prefix and no scale register.  This CPU
test compiles fp8.hip for gfx950 to assembly and checks that every fp8 GEMM
tile kernel issues only that instruction.  The products' values are checked
on the GPU (tests/test_gpu_moe_fp8.py) against the oracle."""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "fe2o3_amd", "csrc")


def test_fp8_gemm_kernels_use_the_unscaled_mfma(tmp_path):
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc) or shutil.which("python3") is None:
        pytest.skip("hipcc not available")
    out = tmp_path / "fp8.s"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                    "-target-feature", "-Xclang", "-packed-fp32-ops", "-munsafe-fp-atomics",
                    "--cuda-device-only", "-S", "-I" + os.path.join(CSRC, "_build"),
                    os.path.join(CSRC, "fp8.hip"), "-o", str(out)],
                   check=True, capture_output=True)
    text = out.read_text()
    bodies = re.findall(r"^(_Z\S*gemm_fp8(?:_128)?_kernel\S*):[^\n]*\n(.*?)^\.Lfunc_end", text,
                        re.S | re.M)
    # 256 x 256 tiles: staged / edge / k tail forms; 128 x 128: two or three
    # stages, whole / edge, tail rounds, k tail
    assert len(bodies) >= 10, [b[0] for b in bodies]
    for name, body in bodies:
        ops = re.findall(r"^\s*(v_mfma\S*)", body, re.M)
        assert ops, name
        assert set(ops) == {"v_mfma_f32_16x16x128_f8f6f4"}, (name, sorted(set(ops)))
