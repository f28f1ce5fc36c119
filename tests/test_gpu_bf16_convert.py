"""bf16 narrowing on the GPU (fe2o3_bf16_from_f32: Bf16::from_f32 of
crates/fe2o3-device/src/half.rs:182-190 over an array) against the CPU
oracle's restatement of the same rule (oracle/common.c
fe2o3o_bf16_from_f32_array), bit for bit.

Every bf16 output of the library (GEMM, fp8 GEMM, flash and MoE epilogues)
goes through the same v_cvt_pk_bf16_f32 narrowing (common.hpp
pack_bf16x2), so this sweep is the parity evidence for replacing the rule
written out in software with the instruction:
  - all 2^32 binary32 patterns, in chunks of 2^28 (pattern p lands in the
    low half of the packed instruction when p is even, the high half when
    odd);
  - a 2^16 x 320-pattern subset (every sign, exponent and top mantissa bit,
    with 320 low halves that hold every rounding case: ties, just below and
    above ties, NaN payloads held only in discarded bits) shifted by one
    element, so each of those patterns also goes through the other half;
  - unaligned arrays (the element-by-element path) and a length that leaves
    a tail.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CHUNK = 1 << 28


def _convert(gpu, bits: np.ndarray, offset: int = 0) -> np.ndarray:
    """bf16 bits of the float32 patterns `bits`, converted on the GPU from
    a buffer placed `offset` float32 elements past an aligned start."""
    from fe2o3_amd import kernels
    host = np.zeros(bits.size + offset, np.uint32)
    host[offset:] = bits
    x = gpu.to_device(host.view(np.float32))
    out = gpu.alloc(bits.size + offset, np.uint16)
    kernels.bf16_from_f32(x.view(offset, bits.size), out.view(offset, bits.size))
    return out.download()[offset:]


def test_bf16_narrowing_every_binary32_pattern(gpu, oracle):
    mismatches = 0
    base = np.arange(CHUNK, dtype=np.uint32)
    for c0 in range(0, 1 << 32, CHUNK):
        bits = base + np.uint32(c0)
        got = _convert(gpu, bits)
        want = oracle.bf16_from_f32(bits.view(np.float32))
        bad = np.nonzero(got != want)[0]
        mismatches += bad.size
        assert bad.size == 0, (hex(int(bits[bad[0]])), hex(int(got[bad[0]])), hex(int(want[bad[0]])))
    assert mismatches == 0


def test_bf16_narrowing_both_halves_and_paths(gpu, oracle):
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lo = np.concatenate([np.arange(0, 64), np.arange(0x7FC0, 0x8040), np.arange(0xFFC0, 0x10000),
                         np.random.default_rng(7).integers(0, 1 << 16, 64)]).astype(np.uint32)
    assert lo.size == 320
    bits = (hi[:, None] | lo[None, :]).ravel()
    want = oracle.bf16_from_f32(bits.view(np.float32))
    for offset in (1, 2, 3):  # shifted by one: the other half; 2, 3: unaligned path
        got = _convert(gpu, bits, offset)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (offset, hex(int(bits[bad[0]])), hex(int(got[bad[0]])))
    tail = bits[:1000003]
    assert np.array_equal(_convert(gpu, tail), want[:1000003])


def test_bf16_narrowing_rejects_length_mismatch(gpu):
    from fe2o3_amd import _lib
    from fe2o3_amd.runtime import Fe2o3Error
    x = gpu.alloc(8, np.float32)
    y = gpu.alloc(7, np.uint16)
    with pytest.raises(Fe2o3Error) as e:
        from fe2o3_amd import kernels
        kernels.bf16_from_f32(x, y)
    assert e.value.status == -2
    assert _lib.lib().fe2o3_bf16_from_f32(None, 0, None, 0, None) == 0
