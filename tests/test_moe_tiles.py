"""CPU check (no GPU): the MoE expert-GEMM work list
(fe2o3_amd/csrc/moe_tiles.hpp, compiled for the host exactly as the gate/up
and down kernels compile it for gfx950) keeps every workgroup's tile inside
the workspace for arbitrary device-resident offsets, and runs every tile of
a consistent routing exactly once over the launch grid."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_moe_tile_list_bounds_and_coverage(tmp_path):
    exe = tmp_path / "moe_tiles_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-o", str(exe),
                    os.path.join(ROOT, "tests", "moe_tiles_check.cpp")], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "failures 0" in r.stdout
