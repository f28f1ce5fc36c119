"""The pipelined general GEMM issues its transposing LDS reads as inline asm
(gemm_pipe::Bf16MmaKN::read, Bf16MmaKN64::read), which the compiler does not see as loads: it
relies on the compiler's own s_waitcnt lgkmcnt for the A read issued before
them.  This CPU test compiles gemm_small.hip for gfx950 to assembly and
replays the instruction streams of gemm_general_pipe_kernel (256x256
tiles) and gemm_general_pipe128_kernel<2>, <3> (128x128, whole grids and
tail rounds), each with whole stages and with a partial last stage, in
text order with in-order LDS
completion: no instruction -- an LDS read's address included -- may read a
VGPR that an LDS read has not yet delivered (no s_waitcnt lgkmcnt covering
it).  The two reads of one inline-asm pair are the case the compiler cannot
see: without early-clobber outputs it may give the first read's destination
the register that holds the second read's address.  Scalar loads share the
counter; the replay ignores them, which only keeps more LDS reads pending
than the hardware would, so the check stays conservative.  The check is
shown to fire on the same stream with its lgkmcnt waits removed."""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "fe2o3_amd", "csrc")


def _regs(tok):
    m = re.match(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _violations(lines):
    pending, bad = [], 0
    for line in lines:
        if not line or line.startswith(".") or line.endswith(":"):
            continue
        op = line.split()[0]
        args = [a.strip() for a in line[len(op):].split(",")]
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", line)
            if m:
                keep = int(m.group(1))
                pending = pending[len(pending) - keep:] if 0 < keep < len(pending) else (
                    [] if keep == 0 else pending)
            continue
        # sources: every operand after the destination; a DS write or atomic
        # without return reads all of its operands (the address first).  An
        # LDS read may name its own destination as its address (it reads the
        # address at issue), but not a destination of an earlier read still
        # in flight
        srcs = set()
        for a in (args if op.startswith("ds_write") else args[1:]):
            srcs |= _regs(a.split()[0] if a else a)
        live = set().union(*pending) if pending else set()
        if srcs & live:
            bad += 1
        if op.startswith("ds_read"):
            pending.append(_regs(args[0]))
        elif op.startswith("ds_"):
            pending.append(set())
    return bad


def test_general_pipe_kernel_lds_reads_are_waited_for(tmp_path):
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc) or shutil.which("python3") is None:
        pytest.skip("hipcc not available")
    out = tmp_path / "gemm_small.s"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                    "-target-feature", "-Xclang", "-packed-fp32-ops", "-munsafe-fp-atomics",
                    "--cuda-device-only", "-S", "-I" + os.path.join(CSRC, "_build"),
                    os.path.join(CSRC, "gemm_small.hip"), "-o", str(out)],
                   check=True, capture_output=True)
    text = out.read_text()
    found = 0
    for m in re.finditer(r"^(_Z\S*gemm_general_pipe\S*kernel\S*):\s*;.*?\n(.*?)\n\s*s_endpgm",
                         text, re.S | re.M):
        name = m.group(1)
        found += 1
        body = [l.split(";")[0].strip() for l in m.group(2).split("\n")]
        assert sum("ds_read_b64_tr_b16" in l for l in body) >= 64, name
        assert _violations(body) == 0, name
        # the check fires when the waits are gone
        stripped = [re.sub(r"lgkmcnt\(\d+\)", "", l) if l.startswith("s_waitcnt") else l
                    for l in body]
        stripped = [l for l in stripped if l.strip() != "s_waitcnt"]
        assert _violations(stripped) > 50, name
    # 256x256, and 128x128 on two and three stages, whole grid or tail; each
    # with whole 64-k stages and with a partial last stage (K tail)
    assert found == 10
