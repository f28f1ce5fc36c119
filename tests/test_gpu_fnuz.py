"""GPU parity of the gfx942 FNUZ fp8 conversions (fe2o3_fp8_fnuz_from_f32 /
fe2o3_fp8_fnuz_to_f32; crates/fe2o3-device/src/fp8.rs:85-95, 193-203) through
the C-ABI, bit-exact against the reference's native gfx942 golden fixture
(tests/golden/fp8_gfx942_rocm.golden) and the CPU oracle (oracle/fp8.c):
every code, every golden narrowing, random bit patterns (NaN payloads,
infinities, f32 subnormals included), unaligned arrays and ragged tails on
the element-at-a-time path, a full-size round trip, and the host-side
errors."""
from __future__ import annotations

import numpy as np
import pytest

from golden import fnuz_golden
from gpu_util import Guarded, assert_same

pytestmark = pytest.mark.gpu

FMTS = [0, 1]  # E4M3 FNUZ, E5M2 FNUZ


def _k():
    from fe2o3_amd import kernels
    return kernels


def _golden():
    return fnuz_golden.load()


@pytest.mark.parametrize("fmt", FMTS)
def test_widen_every_code_matches_golden(gpu, fmt):
    want = np.zeros(256, np.uint32)
    for f, code, bits in _golden()["widen"]:
        if f == fmt:
            want[code] = bits
    q = Guarded(gpu, np.arange(256, dtype=np.uint8))
    x = Guarded(gpu, np.zeros(256, np.float32))
    _k().fp8_fnuz_to_f32(q.body, x.body, fmt)
    assert q.unchanged() and x.guards_intact()
    assert_same(x.download().view(np.uint32), want, "widened bits")


@pytest.mark.parametrize("fmt", FMTS)
def test_narrow_every_golden_case(gpu, fmt):
    cases = [(b, c) for f, _, b, c in _golden()["narrow"] if f == fmt]
    bits = np.array([b for b, _ in cases], np.uint32)
    want = np.array([c for _, c in cases], np.uint8)
    x = Guarded(gpu, bits.view(np.float32))
    q = Guarded(gpu, np.full(bits.size, 0x5A, np.uint8))
    _k().fp8_fnuz_from_f32(x.body, q.body, fmt)
    assert x.unchanged() and q.guards_intact()
    assert_same(q.download(), want, "narrowed codes")


@pytest.mark.parametrize("fmt", FMTS)
def test_pack_records_are_the_little_endian_view(gpu, fmt):
    """Fp8*Fnuzx4 (fp8.rs:435-518): four codes through a device round trip
    (widen, narrow) come back as the golden packed word."""
    packs = [(lanes, word) for f, _, lanes, word in _golden()["pack"] if f == fmt]
    codes = np.array([c for lanes, _ in packs for c in lanes], np.uint8)
    q = gpu.to_device(codes)
    x = gpu.alloc(codes.size, np.float32)
    back = gpu.alloc(codes.size, np.uint8)
    _k().fp8_fnuz_to_f32(q, x, fmt)
    _k().fp8_fnuz_from_f32(x, back, fmt)
    words = back.download().view("<u4")
    assert words.tolist() == [w for _, w in packs]


@pytest.mark.parametrize("fmt", FMTS)
def test_narrow_matches_oracle_on_random_bits(gpu, oracle, fmt):
    rng = np.random.default_rng(70 + fmt)
    n = 1 << 22
    bits = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    top = 240.0 if fmt == 0 else 57344.0
    spread = (rng.standard_normal(n) * np.exp2(rng.uniform(-22, np.log2(top) + 1, n)))
    bits = np.concatenate([bits, spread.astype(np.float32).view(np.uint32),
                           np.array([0, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00000,
                                     0xffc00000, 0x7f800001, 0xff80dead, 1, 0x807fffff],
                                    np.uint32)])
    x = bits.view(np.float32)
    dx = gpu.to_device(x)
    dq = gpu.alloc(x.size, np.uint8)
    _k().fp8_fnuz_from_f32(dx, dq, fmt)
    assert_same(dq.download(), oracle.fnuz_from_f32(x, fmt), "codes")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("n, off", [(1, 0), (15, 0), (17, 0), (4099, 0), (4099, 1),
                                    (4099, 3), (4099, 4), (1000003, 0), (1000003, 4),
                                    (1000003, 5)])
def test_tails_and_unaligned(gpu, oracle, fmt, n, off):
    """Lengths off the 4-element unit and the 4096-element step, and element
    offsets into guarded allocations: offset 4 leaves the f32 array 16-byte
    and the codes 4-byte aligned (the unit path), offsets 1, 3 and 5 take
    the element-at-a-time kernels."""
    rng = np.random.default_rng(n + off)
    x = (rng.standard_normal(n) * 50).astype(np.float32)
    xs = Guarded(gpu, np.concatenate([np.zeros(off, np.float32), x]))
    qs = Guarded(gpu, np.zeros(n + off, np.uint8))
    xv = xs.full.view(64 + off, n)
    qv = qs.full.view(64 + off, n)
    _k().fp8_fnuz_from_f32(xv, qv, fmt)
    want = oracle.fnuz_from_f32(x, fmt)
    got = qs.download()
    assert_same(got[off:], want, "codes")
    assert not got[:off].any() and qs.guards_intact() and xs.unchanged()
    back = Guarded(gpu, np.zeros(n + off, np.float32))
    _k().fp8_fnuz_to_f32(qv, back.full.view(64 + off, n), fmt)
    table = np.array([oracle.fnuz_to_f32_bits(c, fmt) for c in range(256)], np.uint32)
    assert_same(back.download()[off:].view(np.uint32), table[want], "widened")
    assert back.guards_intact()


@pytest.mark.parametrize("fmt", FMTS)
def test_full_size_round_trip(gpu, fmt):
    """2^26 codes: widen then narrow returns every code (0x80 included,
    through its NaN), and narrowing is idempotent on the widened values."""
    n = 1 << 26
    rng = np.random.default_rng(5 + fmt)
    codes = rng.integers(0, 256, n, dtype=np.uint8)
    q = gpu.to_device(codes)
    x = gpu.alloc(n, np.float32)
    q2 = gpu.alloc(n, np.uint8)
    _k().fp8_fnuz_to_f32(q, x, fmt)
    _k().fp8_fnuz_from_f32(x, q2, fmt)
    assert_same(q2.download(), codes, "round trip")
    xb = x.download().view(np.uint32)
    assert np.all(xb[codes == 0x80] == 0xffc00000)
    assert not np.any(xb[codes != 0x80] == 0x80000000)  # no negative zero


def test_host_errors(gpu):
    from fe2o3_amd import _lib
    L = _lib.lib()
    x = gpu.alloc(32, np.float32)
    q = gpu.alloc(32, np.uint8)
    assert L.fe2o3_fp8_fnuz_from_f32(x.ptr, 32, q.ptr, 31, 0, None) == -2
    assert L.fe2o3_fp8_fnuz_to_f32(q.ptr, 32, x.ptr, 31, 1, None) == -2
    assert L.fe2o3_fp8_fnuz_from_f32(x.ptr, 32, q.ptr, 32, 2, None) == -3
    assert L.fe2o3_fp8_fnuz_to_f32(q.ptr, 32, x.ptr, 32, -1, None) == -3
    assert L.fe2o3_fp8_fnuz_from_f32(None, 32, q.ptr, 32, 0, None) == -19
    assert L.fe2o3_fp8_fnuz_to_f32(q.ptr, 32, None, 32, 0, None) == -19
    assert L.fe2o3_fp8_fnuz_from_f32(None, 0, None, 0, 0, None) == 0
    assert L.fe2o3_fp8_fnuz_to_f32(None, 0, None, 0, 1, None) == 0
