"""CPU check (no GPU): the FNUZ fp8 element conversions of
fe2o3_amd/csrc/fp8_fnuz.hpp, compiled for the host exactly as the gfx950
kernels compile them, equal the oracle (oracle/fp8.c, pinned by the
reference's gfx942 golden in tests/test_oracle_fnuz.py) on every f32 input
and every code of both formats."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_fnuz_conversions_equal_the_oracle_on_every_input(tmp_path):
    from oracle import oracle
    oracle.lib()  # builds oracle/liboracle.so when missing
    exe = tmp_path / "fnuz_check"
    odir = os.path.join(ROOT, "oracle")
    subprocess.run(["g++", "-O3", "-std=c++17", "-fopenmp", "-o", str(exe),
                    os.path.join(ROOT, "tests", "fnuz_check.cpp"), "-L" + odir, "-loracle",
                    "-Wl,-rpath," + odir], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600,
                       env={**os.environ, "OMP_NUM_THREADS": str(min(8, os.cpu_count() or 1))})
    assert r.returncode == 0, r.stdout + r.stderr
    assert "failures 0" in r.stdout
