"""The pipelined GEMM tile's LDS swizzle (gemm_pipe::Geo<128>::swz) against
the bank model the rocprofv3 counters fit: a ds_read_b128 is served in four
passes of 16 lanes, {8k .. 8k+7} and {8k+16 .. 8k+23} (k = 0, 1, 4, 5), over
64 banks of 4 bytes.  Under it the two read patterns the tiles use must be
conflict-free: bf16 16x16x32 (lane l reads row l%16, chunk 4s + l/16) and
fp8 16x16x128 (row l%16, chunk 2(l/16) + h), from any 16-row block.  The
model reproduces the three measurements taken with the earlier swizzle
(r ^ (r >> 2)) & 7: bf16 16x16x32 and fp8 32x32x64 free of conflicts, fp8
16x16x128 with 2-way conflicts; the test checks that too, so a formula that
conflicts cannot pass.  The formula is read from the header itself."""
from __future__ import annotations

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "fe2o3_amd", "csrc", "gemm_pipe.hpp")


def header_swizzle():
    text = open(HEADER).read()
    m = re.search(r"if \(ROW_BYTES == 128\) return (.+?);", text)
    assert m, "Geo::swz for 128-byte rows not found"
    expr = re.sub(r"(\d+)u\b", r"\1", m.group(1))
    return lambda r: eval(expr, {}, {"r": r})  # C integer operators read the same in Python


def old_swizzle(r):
    return (r ^ (r >> 2)) & 7


def ways(addr):
    """Most distinct dwords any bank serves in one pass of a ds_read_b128."""
    worst = 1
    for base in (0, 8, 32, 40):
        banks = {}
        for lane in list(range(base, base + 8)) + list(range(base + 16, base + 24)):
            a = addr(lane)
            for w in range(4):
                banks.setdefault((a // 4 + w) % 64, set()).add(a // 4 + w)
        worst = max(worst, max(len(v) for v in banks.values()))
    return worst


def bf16_pattern(swz, s, base):
    return lambda l: (base + l % 16) * 128 + (((4 * s + l // 16) ^ swz(base + l % 16)) << 4)


def fp8_pattern(swz, h, base):
    return lambda l: (base + l % 16) * 128 + (((2 * (l // 16) + h) ^ swz(base + l % 16)) << 4)


def fp8_32x32_pattern(swz, s, h, base):
    return lambda l: (base + l % 32) * 128 + (((4 * s + 2 * (l // 32) + h) ^ swz(base + l % 32)) << 4)


def worst_ways(swz):
    bf16 = max(ways(bf16_pattern(swz, s, b)) for s in (0, 1) for b in range(0, 288, 16))
    fp8 = max(ways(fp8_pattern(swz, h, b)) for h in (0, 1) for b in range(0, 256, 16))
    return bf16, fp8


def test_swizzle_is_a_permutation_of_each_row():
    swz = header_swizzle()
    for r in range(512):
        assert 0 <= swz(r) < 8
        assert sorted(c ^ swz(r) for c in range(8)) == list(range(8))


def test_header_swizzle_is_conflict_free_for_both_read_patterns():
    assert worst_ways(header_swizzle()) == (1, 1)


def test_model_reproduces_the_measured_counters_of_the_earlier_swizzle():
    # bf16 and fp8 32x32x64 measured SQ_LDS_BANK_CONFLICT = 0, fp8 16x16x128
    # measured 2-way conflicts (3.4e7 cycles at 8192^3)
    assert worst_ways(old_swizzle) == (1, 2)
    f32 = max(ways(fp8_32x32_pattern(old_swizzle, s, h, b))
              for s in (0, 1) for h in (0, 1) for b in range(0, 256, 32))
    assert f32 == 1


def test_lane_offsets_cover_every_row_block():
    """The policies keep lane offsets per row-block parity at most
    (Fp8Mma16: l.a[i & 1]) and add row blocks of 16 rows as immediates: the
    swizzle of row 16i + r may depend on i only through i & 1."""
    swz = header_swizzle()
    for r in range(16):
        for parity in (0, 1):
            assert len({swz(16 * i + r) for i in range(parity, 64, 2)}) == 1
