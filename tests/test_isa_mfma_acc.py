"""The MFMAs of the pipelined GEMM tile are inline asm (gemm_pipe::Bf16Mma),
hidden from the compiler's hazard recognizer, so their accumulators must be
touched by nothing but MFMAs until the tile's finish() has put its wait
states in.  The MoE expert kernels' 288-row form keeps a ninth row block's
accumulators in VGPRs, which the compiler could otherwise copy or reuse.
This CPU test compiles moe.hip for gfx950 to assembly and checks, for
gate_up_kernel and down_kernel:
  - the VGPRs written by MFMAs are read or written by no other instruction
    between the first and the last of those MFMAs;
  - every other instruction that reads an accumulator (an AGPR, or those
    VGPRs after their last MFMA) comes at least 18 wait states (an
    instruction each, s_nop N counting N + 1) after the last MFMA before it
    in program order, the most a 16-pass MFMA's result needs before a VALU
    or memory instruction reads it.
Both checks are shown to fire on the same instruction stream with a planted
copy of an accumulator and with the s_nop wait states removed."""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "fe2o3_amd", "csrc")
WAIT_STATES = 18


def _regs(line):
    out = set()
    for m in re.finditer(r"\b([va])\[(\d+):(\d+)\]", line):
        out |= {(m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1)}
    for m in re.finditer(r"\b([va])(\d+)\b", line):
        out.add((m.group(1), int(m.group(2))))
    return out


def _is_insn(line):
    return bool(line) and not line.startswith(".") and not line.endswith(":")


def _waits(line):
    m = re.match(r"s_nop\s+(\d+)", line)
    return int(m.group(1)) + 1 if m else 1


def _check(body):
    """(MFMAs with VGPR accumulators, span violations, fewest wait states
    between an MFMA and a later non-MFMA read of an accumulator)"""
    is_mfma = [l.startswith("v_mfma") for l in body]
    vdst = [i for i, l in enumerate(body) if is_mfma[i] and l.split()[1].startswith("v[")]
    accs = set()
    for i in vdst:
        accs |= _regs(body[i].split(",")[0])
    span_bad = 0
    if vdst:
        for i in range(vdst[0], vdst[-1] + 1):
            if _is_insn(body[i]) and not is_mfma[i] and _regs(body[i]) & accs:
                span_bad += 1
    fewest = 10 ** 9
    since = None
    first_after = True
    for i, line in enumerate(body):
        if not _is_insn(line):
            continue
        if is_mfma[i]:
            since = 0
            continue
        regs = _regs(line)
        reads_agpr = any(r[0] == "a" for r in regs)
        reads_vacc = bool(vdst) and i > vdst[-1] and first_after and bool(regs & accs)
        if reads_vacc:
            first_after = False
        if since is not None and (reads_agpr or reads_vacc):
            fewest = min(fewest, since)
        if since is not None:
            since += _waits(line)
    return len(vdst), span_bad, fewest


def _bodies(text, names):
    out = {}
    for name in names:
        m = re.search(r"^(_Z\S*%s\S*):[^\n]*\n(.*?)^\.Lfunc_end" % name, text, re.S | re.M)
        assert m, name
        out[name] = [l.split(";")[0].strip() for l in m.group(2).split("\n")]
    return out


def test_moe_kernels_accumulators_untouched_until_waited(tmp_path):
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc) or shutil.which("python3") is None:
        pytest.skip("hipcc not available")
    out = tmp_path / "moe.s"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                    "-target-feature", "-Xclang", "-packed-fp32-ops", "-munsafe-fp-atomics",
                    "--cuda-device-only", "-S", "-I" + os.path.join(CSRC, "_build"),
                    os.path.join(CSRC, "moe.hip"), "-o", str(out)],
                   check=True, capture_output=True)
    bodies = _bodies(out.read_text(), ["gate_up_kernelILb1", "gate_up_kernelILb0", "down_kernel"])
    for name, body in bodies.items():
        n_vacc, span_bad, fewest = _check(body)
        # the 288-row form: 8 MFMAs per substep into VGPRs, in every unrolled step
        assert n_vacc >= 32, (name, n_vacc)
        assert span_bad == 0, name
        assert fewest >= WAIT_STATES, (name, fewest)
        # the checks fire: a copy of a VGPR accumulator planted inside the span ...
        vdst = [i for i, l in enumerate(body)
                if l.startswith("v_mfma") and l.split()[1].startswith("v[")]
        acc = re.match(r"v_mfma\S*\s+v\[(\d+):", body[vdst[-1]]).group(1)
        planted = body[:vdst[-1]] + [f"v_mov_b32 v250, v{acc}"] + body[vdst[-1]:]
        assert _check(planted)[1] > 0, name
        # ... and the epilogue without its wait states
        no_nops = [l for l in body if not l.startswith("s_nop")]
        assert _check(no_nops)[2] < WAIT_STATES, name
