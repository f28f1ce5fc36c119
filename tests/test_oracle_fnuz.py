"""CPU pins of the oracle's gfx942 FNUZ fp8 conversions (oracle/fp8.c,
restating crates/fe2o3-device/src/fp8.rs:296-381):
  * every record of the reference's native gfx942 golden fixture
    (512 widenings, 2092 narrowings, 14 packings);
  * the reference's own unit tests (crates/fe2o3-device/tests/fp8_api.rs):
    constants, every encoding round-trips, NaN / infinity / overflow /
    underflow / negative zero canonicalization;
  * brute force: narrowing equals the nearest of the 255 finite values
    (ties to the even code), saturating above the largest, on boundary,
    random and special f32 inputs -- independent of the oracle's shift
    arithmetic, so a wrong bias, a dropped carry or a tie rounded away from
    even fails it."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))

from oracle import oracle  # noqa: E402
import fnuz_golden  # noqa: E402

MAX_BITS = {0: 0x43700000, 1: 0x47600000}


def _f(bits):
    return np.array([bits], np.uint32).view(np.float32)[0]


def test_golden_fixture_shape():
    g = fnuz_golden.load()
    assert len(g["widen"]) == 512 and len(g["narrow"]) == 2092 and len(g["pack"]) == 14
    assert g["meta"]["target"] == "gfx942" and g["meta"]["rounding"] == "rne"
    assert g["meta"]["saturation"] == "satfinite" and g["meta"]["fnuz-nan-f32"] == "ffc00000"


def test_oracle_matches_every_golden_record():
    g = fnuz_golden.load()
    for fmt, code, bits in g["widen"]:
        assert oracle.fnuz_to_f32_bits(code, fmt) == bits, (fmt, hex(code))
    for fmt, case, bits, code in g["narrow"]:
        assert oracle.fnuz_from_f32_bits(bits, fmt) == code, (fmt, case)
    for fmt, case, lanes, word in g["pack"]:
        # the packed x4 value is the little-endian view of four codes
        assert int(np.array(lanes, np.uint8).view("<u4")[0]) == word, (fmt, case)


def test_reference_unit_test_values():
    # fp8_api.rs: constants and doc examples
    assert oracle.fnuz_from_f32_bits(0x3fc00000, 0) == 0x44  # 1.5
    assert _f(oracle.fnuz_to_f32_bits(0x7f, 0)) == 240.0
    assert _f(oracle.fnuz_to_f32_bits(0xff, 0)) == -240.0
    assert _f(oracle.fnuz_to_f32_bits(0x08, 0)) == 2.0 ** -7
    assert _f(oracle.fnuz_to_f32_bits(0x01, 0)) == 2.0 ** -10
    assert _f(oracle.fnuz_to_f32_bits(0x7f, 1)) == 57344.0
    assert _f(oracle.fnuz_to_f32_bits(0xff, 1)) == -57344.0
    assert _f(oracle.fnuz_to_f32_bits(0x04, 1)) == 2.0 ** -15
    assert _f(oracle.fnuz_to_f32_bits(0x01, 1)) == 2.0 ** -17
    for fmt in (0, 1):
        assert _f(oracle.fnuz_to_f32_bits(0x40, fmt)) == 1.0
        assert oracle.fnuz_to_f32_bits(0x80, fmt) == 0xffc00000
        # every encoding round-trips
        for raw in range(256):
            bits = oracle.fnuz_to_f32_bits(raw, fmt)
            assert oracle.fnuz_from_f32_bits(bits, fmt) == raw, (fmt, raw)
        # NaN, infinities -> 0x80; -0 -> 0x00
        for bits in (0x7fc00000, 0x7f800001, 0xffc01234, 0x7f800000, 0xff800000):
            assert oracle.fnuz_from_f32_bits(bits, fmt) == 0x80
        assert oracle.fnuz_from_f32_bits(0x80000000, fmt) == 0
    f2b = lambda v: int(np.array([v], np.float32).view(np.uint32)[0])  # noqa: E731
    assert oracle.fnuz_from_f32_bits(f2b(241.0), 0) == 0x7f
    assert oracle.fnuz_from_f32_bits(f2b(-241.0), 0) == 0xff
    assert oracle.fnuz_from_f32_bits(f2b(60000.0), 1) == 0x7f
    assert oracle.fnuz_from_f32_bits(f2b(-60000.0), 1) == 0xff
    assert oracle.fnuz_from_f32_bits(f2b(2.0 ** -11), 0) == 0
    assert oracle.fnuz_from_f32_bits(f2b(2.0 ** -18), 1) == 0


def _brute(bits: np.ndarray, fmt: int) -> np.ndarray:
    """Nearest finite FNUZ value by search over the decode table, from the
    format's definition: code c != 0x80 has value (-1)^s m 2^k with
    m = frac (exponent field 0) or 2^mb + frac, k = max(ef, 1) - bias - mb."""
    mb, bias = (3, 8) if fmt == 0 else (2, 16)
    codes = np.array([c for c in range(256) if c != 0x80], np.int64)
    ef = (codes & 0x7f) >> mb
    frac = codes & ((1 << mb) - 1)
    m = np.where(ef == 0, frac, frac + (1 << mb)).astype(np.float64)
    vals = m * np.exp2(np.maximum(ef, 1) - bias - mb) * np.where(codes & 0x80, -1.0, 1.0)
    order = np.argsort(vals, kind="stable")
    # 0x00 and nothing else is zero (0x80 is excluded)
    vals, codes = vals[order], codes[order]
    with np.errstate(invalid="ignore"):  # signaling NaNs
        x = bits.view(np.float32).astype(np.float64)
    out = np.empty(bits.size, np.int64)
    nan = ~np.isfinite(x)
    vmax = vals[-1]
    sat = np.abs(x) > vmax
    xi = np.clip(x, vals[0], vals[-1])
    hi = np.clip(np.searchsorted(vals, xi), 1, vals.size - 1)
    lo = hi - 1
    dlo, dhi = xi - vals[lo], vals[hi] - xi
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((codes[hi] & 1) == 0))
    out[:] = np.where(pick_hi, codes[hi], codes[lo])
    out[sat] = np.where(x[sat] > 0, 0x7f, 0xff)
    out[nan] = 0x80
    return out.astype(np.uint8)


@pytest.mark.parametrize("fmt", [0, 1])
def test_oracle_narrowing_is_nearest_even_by_brute_force(fmt):
    rng = np.random.default_rng(20 + fmt)
    g = fnuz_golden.load()
    boundary = np.array([b for f, _, b, _ in g["narrow"] if f == fmt], np.uint32)
    # random bit patterns, plus random values spread over the format's range
    rnd = rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32)
    top = 240.0 if fmt == 0 else 57344.0
    spread = (rng.standard_normal(200_000) * np.exp2(rng.uniform(-20, np.log2(top) + 1, 200_000)))
    spread = spread.astype(np.float32).view(np.uint32)
    # every midpoint between adjacent finite values, and its neighbours
    table = np.array([oracle.fnuz_to_f32_bits(c, fmt) for c in range(256) if c != 0x80],
                     np.uint32).view(np.float32).astype(np.float64)
    table = np.unique(table)
    mids = ((table[1:] + table[:-1]) / 2).astype(np.float32)  # exact: one more bit
    mid_bits = mids.view(np.uint32)
    near = np.concatenate([mid_bits, mid_bits + 1, mid_bits - 1])
    specials = np.array([0, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00000, 0xffc00000,
                         0x7f800001, 0x00000001, 0x807fffff, MAX_BITS[fmt],
                         MAX_BITS[fmt] + 1, MAX_BITS[fmt] | 0x80000000], np.uint32)
    bits = np.concatenate([boundary, rnd, spread, near, specials]).astype(np.uint32)
    got = np.array([oracle.fnuz_from_f32_bits(int(b), fmt) for b in bits[:4000]], np.uint8)
    assert np.array_equal(got, _brute(bits[:4000], fmt))
    x = bits.view(np.float32)
    assert np.array_equal(oracle.fnuz_from_f32(x, fmt), _brute(bits, fmt))


def test_brute_force_check_fires_on_a_wrong_tie_rule():
    """The brute-force reference catches a plausible mistake: ties rounded
    away from zero instead of to even."""
    bits = np.array([0x3a000000, 0x3ac00000, 0x3f880000], np.uint32)  # ties
    exact = _brute(bits, 0)
    assert list(exact) == [0x00, 0x02, 0x40]
    away = [0x01, 0x02, 0x41]  # 2^-11 -> 2^-10, 1.0625 -> 1.125
    assert list(exact) != away
