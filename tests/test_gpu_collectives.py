"""GPU parity tests for the wave64 collectives, the workgroup-sync profiles and
the on-device routing-output consistency check, through the C-ABI, against
the CPU oracle (oracle/sync.c).

All of it is bit-exact: the collectives reproduce the oracle's fixed round
order for any finite input (not only the reference's integral corpus), the
integer reduction and atomic are exact, and the routing check reports the
same first failing relation as the reference's sequential check.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import Guarded

pytestmark = pytest.mark.gpu

FULL = 0xFFFFFFFFFFFFFFFF
REFERENCE_MASKS = [FULL, 0, 0xAAAAAAAAAAAAAAAA,
                   (1 << 0) | (1 << 1) | (1 << 31) | (1 << 32) | (1 << 62) | (1 << 63),
                   (1 << 19) - 1, (1 << 0) | (1 << 3) | (1 << 8) | (1 << 34) | (1 << 63)]


def _k():
    from fe2o3_amd import kernels
    return kernels


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32).tolist()


def _run64(gpu, x, mask):
    gx = Guarded(gpu, np.asarray(x, np.float32))
    outs = [Guarded(gpu, np.full(64, np.nan, np.float32)) for _ in range(3)]
    _k().wave64_collectives_v1(gx.body, mask, *[o.body for o in outs])
    assert gx.unchanged() and all(o.guards_intact() for o in outs)
    return [o.download() for o in outs]


@pytest.mark.parametrize("mask", REFERENCE_MASKS)
def test_wave64_reference_masks_bit_exact(gpu, oracle, mask):
    """examples/wave64_collectives_v1/tests/gfx942_hardware.rs:252-254,417-422:
    the hardware corpus and masks."""
    x = np.array([((lane * 13 + 5) % 31) - 15 for lane in range(64)], np.float32)
    rc, *ref = oracle.wave64_collectives(x, mask)
    assert rc == 0
    for got, want in zip(_run64(gpu, x, mask), ref):
        assert _bits(got) == _bits(want)


def test_wave64_signed_zero_endpoints(gpu, oracle):
    x = np.zeros(64, np.float32)
    x[0], x[1], x[63] = -0.0, -1024.0, 1024.0
    mask = (1 << 0) | (1 << 1) | (1 << 63)
    _, *ref = oracle.wave64_collectives(x, mask)
    for got, want in zip(_run64(gpu, x, mask), ref):
        assert _bits(got) == _bits(want)


@pytest.mark.parametrize("seed", range(6))
def test_wave64_any_finite_input_bit_exact(gpu, oracle, seed):
    """Non-integral inputs of mixed magnitude: the device rounds in the
    oracle's order, so every bit matches."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(64) * 10.0 ** rng.integers(-3, 4, 64)).astype(np.float32)
    mask = int(rng.integers(0, 2**63)) * 2 + int(rng.integers(0, 2))
    _, *ref = oracle.wave64_collectives(x, mask, admit=False)
    for got, want in zip(_run64(gpu, x, mask), ref):
        assert _bits(got) == _bits(want)


def test_wave64_rejects_wrong_lengths(gpu):
    from fe2o3_amd.runtime import Fe2o3Error
    a = gpu.alloc(63, np.float32)
    b = [gpu.alloc(64, np.float32) for _ in range(3)]
    with pytest.raises(Fe2o3Error) as e:
        _k().wave64_collectives_v1(a, FULL, *b)
    assert e.value.status == -2


@pytest.mark.parametrize("rows", [1, 5, 4096 + 3])
def test_wave64_rows_bit_exact(gpu, oracle, rows):
    rng = np.random.default_rng(rows)
    x = rng.standard_normal((rows, 64)).astype(np.float32)
    masks = rng.integers(0, 2**63, rows, dtype=np.uint64) * np.uint64(2) + \
        rng.integers(0, 2, rows, dtype=np.uint64)
    masks[0] = np.uint64(FULL)
    if rows > 1:
        masks[1] = np.uint64(0)
    gx, gm = gpu.to_device(x.ravel()), gpu.to_device(masks)
    outs = [Guarded(gpu, np.full(rows * 64, np.nan, np.float32)) for _ in range(3)]
    _k().wave64_collectives_rows(gx, gm, *[o.body for o in outs], rows)
    got = [o.download().reshape(rows, 64) for o in outs]
    assert all(o.guards_intact() for o in outs)
    sample = sorted(set([0, rows - 1] + list(rng.integers(0, rows, 200))))
    for r in sample:
        _, *ref = oracle.wave64_collectives(x[r], int(masks[r]), admit=False)
        for g, want in zip(got, ref):
            assert _bits(g[r]) == _bits(want), r


def _reduction_vectors():  # examples/workgroup_sync_v1/src/vectors.rs:31-70
    return [[0] * 64, [1000 if l % 2 == 0 else -999 for l in range(64)],
            [l - 32 for l in range(64)], [l * 7 if l % 11 == 0 else 0 for l in range(64)]]


@pytest.mark.parametrize("case", range(4))
def test_lds_reduce_reference_vectors(gpu, oracle, case):
    values = _reduction_vectors()[case]
    rc, want = oracle.lds_reduce_i32(values)
    assert rc == 0
    out = Guarded(gpu, np.array([0x5A5A5A5A], np.int32))
    _k().lds_reduce_i32_v1(gpu.to_device(np.array(values, np.int32)), out.body)
    assert out.guards_intact() and int(out.download()[0]) == want


def test_lds_reduce_random_and_wrapping(gpu, oracle):
    rng = np.random.default_rng(11)
    for _ in range(8):
        v = rng.integers(-(2**24), 2**24, 64, dtype=np.int64).astype(np.int32)
        out = gpu.alloc(1, np.int32)
        _k().lds_reduce_i32_v1(gpu.to_device(v), out)
        assert int(out.download()[0]) == oracle.lds_reduce_i32(v)[1]
    # outside the admitted range the device sum wraps (two's complement)
    v = np.full(64, 2**26, np.int32)
    out = gpu.alloc(1, np.int32)
    _k().lds_reduce_i32_v1(gpu.to_device(v), out)
    assert int(out.download()[0]) == ((64 * 2**26 + 2**31) % 2**32) - 2**31


def _atomic_vectors():  # examples/workgroup_sync_v1/src/vectors.rs:72-109
    ramp = list(range(64))
    return [(17, ramp, [0] * 64), (0, ramp, [1] * 64),
            (11, ramp, [int(l % 2 == 0) for l in range(64)]),
            (1000, ramp, [int(l % 13 == 0) for l in range(64)])]


@pytest.mark.parametrize("case", range(4))
def test_scoped_atomic_reference_vectors(gpu, oracle, case):
    initial, values, eligible = _atomic_vectors()[case]
    rc, want = oracle.atomic_add_u32(initial, values, eligible)
    assert rc == 0
    target = Guarded(gpu, np.array([initial], np.uint32))
    _k().scoped_atomic_add_u32_v1(gpu.to_device(np.array(values, np.uint32)),
                                  gpu.to_device(np.array(eligible, np.uint32)), target.body)
    assert target.guards_intact() and int(target.download()[0]) == want


# ---- routing output consistency on the device ------------------------------------------

ORACLE_KEYS = {"top2": "top2_experts", "requested": "requested_counts",
               "admitted": "admitted_counts", "offsets": "expert_offsets",
               "slots": "route_slots", "permutation": "permutation", "inverse": "inverse"}


def _device_check(gpu, outs, tokens, experts, capacity):
    routing = {k: gpu.to_device(np.ascontiguousarray(outs[v], np.uint32))
               for k, v in ORACLE_KEYS.items()}
    rec = Guarded(gpu, np.full(4, 0xDEADBEEF, np.uint32))
    _k().moe_routing_check(routing, tokens, experts, capacity, rec.body)
    assert rec.guards_intact()
    for k, v in ORACLE_KEYS.items():  # inputs untouched
        assert routing[k].download().tolist() == np.asarray(outs[v]).tolist()
    r = rec.download()
    return int(r[0]), int(r[1]), int(r[2]), int(r[3])


def _oracle_check(oracle, outs, tokens, experts, capacity):
    kind, index, expected, actual = oracle.moe_routing_check(outs, tokens, experts, capacity)
    return oracle.ROUTING_CHECK_KINDS.index(kind), index, expected, actual


def _mutations(outs, rng, routes, experts, n):
    keys = list(ORACLE_KEYS.values())
    for _ in range(n):
        m = {k: np.array(v, np.uint32) for k, v in outs.items()}
        for _ in range(int(rng.integers(1, 3))):
            key = keys[int(rng.integers(0, len(keys)))]
            i = int(rng.integers(0, m[key].size))
            choice = int(rng.integers(0, 5))
            if choice == 0:
                m[key][i] = 0xFFFFFFFF
            elif choice == 1:
                m[key][i] = int(rng.integers(0, routes + 2))
            elif choice == 2:
                m[key][i] = int(rng.integers(0, experts + 1))
            elif choice == 3:
                m[key][i] = (int(m[key][i]) + 1) & 0xFFFFFFFF
            else:
                j = int(rng.integers(0, m[key].size))
                m[key][i], m[key][j] = m[key][j], m[key][i]
        yield m


@pytest.mark.parametrize("tokens,experts,capacity", [(8, 4, 4), (4096, 8, 0xFFFFFFFF),
                                                     (4096, 8, 1000), (777, 64, 30),
                                                     (12288, 16, 0xFFFFFFFF),
                                                     (20000, 8, 0xFFFFFFFF), (15000, 64, 300)])
def test_routing_check_matches_oracle_on_mutations(gpu, oracle, tokens, experts, capacity):
    """The router's own outputs are consistent; random one- and two-element
    corruptions of them (sentinels, in- and out-of-range values, swaps,
    off-by-one) report exactly the oracle's first failing relation.  Up to
    1024 tokens one workgroup checks; above, the check runs over workgroups
    of 256 tokens on stream-ordered scratch."""
    rng = np.random.default_rng(tokens + experts)
    rc, outs = oracle.moe_top2_route(rng.standard_normal((tokens, experts)).astype(np.float32),
                                     tokens, experts, capacity)
    assert rc == 0
    assert _device_check(gpu, outs, tokens, experts, capacity) == (0, 0, 0, 0)
    kinds = set()
    for m in _mutations(outs, rng, 2 * tokens, experts, 60 if tokens <= 4096 else 20):
        want = _oracle_check(oracle, m, tokens, experts, capacity)
        assert _device_check(gpu, m, tokens, experts, capacity) == want
        kinds.add(want[0])
    assert len(kinds) >= 5


def test_routing_check_reference_mutations(gpu, oracle):
    """moe_routing_expert_bridge_v1.rs:738-851 on the device: the base
    routing of every token to experts (0, 1), then each named mutation."""
    logits = np.zeros((8, 4), np.float32)
    logits[:, 0], logits[:, 1] = 2.0, 1.0
    _, base = oracle.moe_top2_route(logits, 8, 4, 4)
    cases = [("expert_offsets", 2, 3), ("admitted_counts", 0, 5), ("route_slots", 8, 0),
             ("inverse", 8, 0), ("permutation", 8, 0), ("route_slots", 0, 16),
             ("permutation", 0, 2), ("inverse", 0, 1), ("requested_counts", 0, 7),
             ("top2_experts", 5, 4), ("top2_experts", 5, 0),
             ("permutation", 9, 0), ("permutation", 15, 0)]
    for key, i, value in cases:
        m = {k: np.array(v, np.uint32) for k, v in base.items()}
        m[key][i] = value
        want = _oracle_check(oracle, m, 8, 4, 4)
        assert want[0] != 0, (key, i)
        assert _device_check(gpu, m, 8, 4, 4) == want, (key, i)


@pytest.mark.parametrize("tokens,capacity,ends,random", [(4096, 700, 130, 40),
                                                         (20000, 3000, 30, 20)])
def test_routing_check_every_permutation_tail_slot(gpu, oracle, tokens, capacity, ends, random):
    """A capacity-limited routing (8 experts, so the permutation has a long
    sentinel tail): a non-sentinel value planted in each tail slot in turn
    is reported as PermutationTail at that slot, as the oracle reports it
    (both sizes run the many-workgroup check: 16 and 79 workgroups)."""
    experts = 8
    rng = np.random.default_rng(11)
    rc, base = oracle.moe_top2_route(rng.standard_normal((tokens, experts)).astype(np.float32),
                                     tokens, experts, capacity)
    assert rc == 0
    accepted = int(base["expert_offsets"][-1])
    assert accepted < 2 * tokens - 200
    tail = list(range(accepted, 2 * tokens))
    picks = tail[:ends] + tail[-ends:] + [int(x) for x in rng.choice(tail, random, replace=False)]
    for s in picks:
        m = {k: np.array(v, np.uint32) for k, v in base.items()}
        m["permutation"][s] = 3
        want = _oracle_check(oracle, m, tokens, experts, capacity)
        assert want[0] == 18 and want[1] == s, (s, want)
        assert _device_check(gpu, m, tokens, experts, capacity) == want, s


@pytest.mark.parametrize("tokens,rounds", [(64, 20), (13000, 4)])
def test_routing_check_garbage_payloads_are_safe(gpu, oracle, tokens, rounds):
    """Arbitrary arrays (ids, offsets and slots far out of range) read only
    in bounds and still report the oracle's first error (13000 tokens: the
    many-workgroup check)."""
    rng = np.random.default_rng(5)
    experts = 8
    for _ in range(rounds):
        outs = {"top2_experts": rng.integers(0, experts + 2, 2 * tokens, dtype=np.uint32),
                "requested_counts": rng.integers(0, 40, experts, dtype=np.uint32),
                "admitted_counts": rng.integers(0, 40, experts, dtype=np.uint32),
                "expert_offsets": np.sort(rng.integers(0, 300, experts + 1)).astype(np.uint32),
                "route_slots": rng.integers(0, 2**32, 2 * tokens, dtype=np.uint64).astype(np.uint32),
                "permutation": rng.integers(0, 2**32, 2 * tokens, dtype=np.uint64).astype(np.uint32),
                "inverse": rng.integers(0, 300, 2 * tokens, dtype=np.uint32)}
        assert _device_check(gpu, outs, tokens, experts, 16) == \
            _oracle_check(oracle, outs, tokens, experts, 16)
    # valid ids, counts and offsets from the router; random slot arrays, so
    # the slot, permutation and tail phases see arbitrary values
    for _ in range(rounds):
        _, outs = oracle.moe_top2_route(rng.standard_normal((tokens, experts)).astype(np.float32),
                                        tokens, experts, 12)
        for key in ("route_slots", "permutation", "inverse"):
            if rng.integers(0, 2):
                outs[key] = rng.integers(0, 2 * tokens + 3, 2 * tokens, dtype=np.uint32)
        assert _device_check(gpu, outs, tokens, experts, 12) == \
            _oracle_check(oracle, outs, tokens, experts, 12)
