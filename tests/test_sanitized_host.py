"""CPU checks (no GPU) of host-side C++ under AddressSanitizer and
UndefinedBehaviorSanitizer.

- The code-object inspector (fe2o3_amd/csrc/codeobj_inspect.hpp) on the
  embedded gfx950 code object and on truncated and mutated copies of it: no
  read outside the buffer, no undefined arithmetic, whatever the bytes.
- The MoE expert tile list (fe2o3_amd/csrc/moe_tiles.hpp) on arbitrary
  device-resident offsets (tests/moe_tiles_check.cpp).
- The non-finite report's bookkeeping (fe2o3_amd/csrc/status_track.hpp).
- The pipelined GEMMs' launch plan and tile orders for the CU and XCD counts
  a device may report (fe2o3_amd/csrc/tile_plan.hpp,
  tests/tile_plan_check.cpp).

Each program is built with g++ -fsanitize=address,undefined
-fno-sanitize-recover=all, so the first finding aborts it with a nonzero
exit status and the sanitizer's report on stderr."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
       "-g", "-O1", "-std=c++17"]
CODE_OBJECT = os.path.join(ROOT, "fe2o3_amd", "csrc", "_build", "tiled_gemm_lds_v1.co")


def _build_and_run(tmp_path, src, args=(), timeout=600):
    exe = tmp_path / os.path.splitext(os.path.basename(src))[0]
    subprocess.run(["g++", *SAN, "-o", str(exe), os.path.join(ROOT, "tests", src)], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=timeout, env=env)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    return r.stdout


def test_codeobj_inspector_sanitized(tmp_path):
    if not os.path.exists(CODE_OBJECT):
        pytest.fail(f"{CODE_OBJECT} is missing: build the library first "
                    "(python -c 'import __graft_entry__ as g; g.build()')")
    out = _build_and_run(tmp_path, "codeobj_inspect_check.cpp", [CODE_OBJECT])
    assert "failures 0" in out, out
    runs = int(out.split("runs ")[1].split()[0])
    assert runs > 40000, out


def test_moe_tiles_sanitized(tmp_path):
    out = _build_and_run(tmp_path, "moe_tiles_check.cpp")
    assert "failures 0" in out, out


def test_status_tracker_sanitized(tmp_path):
    out = _build_and_run(tmp_path, "status_check.cpp")
    assert "failures 0" in out, out


def test_tile_plan_sanitized(tmp_path):
    out = _build_and_run(tmp_path, "tile_plan_check.cpp")
    assert "failures 0" in out, out
