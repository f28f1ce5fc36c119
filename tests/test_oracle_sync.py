"""CPU oracle pins for the wave64 collectives, the workgroup-sync profiles and
the routing-output consistency check, against the reference's own tests:

- examples/wave64_collectives_v1/tests/oracle.rs:6-95 (corpus, masks, closed
  forms, signed zero, admission);
- examples/workgroup_sync_v1/src/vectors.rs:31-109 (named vectors with their
  expected results);
- crates/fe2o3-host/src/moe_routing_expert_bridge_v1.rs:673-870 (the
  reference candidate builder and its hostile mutations with named errors).
"""
import numpy as np
import pytest

from oracle import oracle as O

FULL = 0xFFFFFFFFFFFFFFFF


def _corpus():  # examples/wave64_collectives_v1/tests/oracle.rs:6-8
    return np.array([((lane * 5 + 3) % 17) - 8 for lane in range(64)], np.float32)


@pytest.mark.parametrize("mask", [0, (1 << 19) - 1,
                                  (1 << 0) | (1 << 3) | (1 << 8) | (1 << 34) | (1 << 63),
                                  0xAAAAAAAAAAAAAAAA, FULL,
                                  (1 << 0) | (1 << 1) | (1 << 31) | (1 << 32) | (1 << 62) | (1 << 63)])
def test_wave64_masks_match_closed_form(mask):
    """oracle.rs:24-48: active lanes hold the masked total and their exact
    prefixes; inactive lanes hold +0 in all three outputs."""
    x = _corpus()
    rc, red, inc, exc = O.wave64_collectives(x, mask)
    assert rc == O.OK
    active = [(mask >> lane) & 1 for lane in range(64)]
    total = sum(float(x[lane]) for lane in range(64) if active[lane])
    prefix = 0.0
    for lane in range(64):
        if not active[lane]:
            for out in (red, inc, exc):
                assert out[lane].view(np.uint32) == 0  # +0 bits
        else:
            assert red[lane] == total
            assert exc[lane] == prefix
            prefix += float(x[lane])
            assert inc[lane] == prefix


def test_wave64_signed_zero_and_endpoints():
    """oracle.rs:77-95."""
    x = np.zeros(64, np.float32)
    x[0], x[1], x[63] = -0.0, -1024.0, 1024.0
    mask = (1 << 0) | (1 << 1) | (1 << 63)
    rc, red, inc, exc = O.wave64_collectives(x, mask)
    assert rc == O.OK
    assert red[0] == 0.0
    assert exc[0].view(np.uint32) == 0
    assert inc[1] == -1024.0 and exc[63] == -1024.0 and inc[63] == 0.0


@pytest.mark.parametrize("bad,rc", [(np.nan, O.ERR_NONFINITE), (np.inf, O.ERR_NONFINITE),
                                    (0.5, O.ERR_ALPHABET), (1025.0, O.ERR_ALPHABET),
                                    (-1025.0, O.ERR_ALPHABET)])
def test_wave64_admission_preserves_outputs(bad, rc):
    """oracle.rs:97-156: each invalid input is rejected with the outputs
    untouched (NaN-filled here)."""
    x = _corpus()
    x[17] = bad
    got, red, inc, exc = O.wave64_collectives(x, FULL)
    assert got == rc
    assert np.isnan(red).all() and np.isnan(inc).all() and np.isnan(exc).all()


def test_wave64_fixed_order_differs_from_sequential_sums():
    """The rounds fix the summation order: on non-integral data the butterfly
    reduction differs from a left-to-right sum in some lanes' bits, while
    staying within f32 rounding of the f64 sum.  (The GPU test then checks
    the device reproduces the oracle's order bit for bit.)"""
    rng = np.random.default_rng(7)
    differs = 0
    for _ in range(50):
        x = rng.standard_normal(64).astype(np.float32)
        _, red, inc, _ = O.wave64_collectives(x, FULL, admit=False)
        seq = np.float32(0)
        for v in x:
            seq = np.float32(seq + v)
        differs += red[0] != seq
        exact = float(np.sum(x.astype(np.float64)))
        assert abs(float(red[0]) - exact) <= 64 * 2**-23 * np.abs(x).sum()
        assert abs(float(inc[63]) - exact) <= 64 * 2**-23 * np.abs(x).sum()
    assert differs > 0


def _reduction_vectors():  # examples/workgroup_sync_v1/src/vectors.rs:31-70
    alt = [1000 if lane % 2 == 0 else -999 for lane in range(64)]
    ramp = [lane - 32 for lane in range(64)]
    sparse = [lane * 7 if lane % 11 == 0 else 0 for lane in range(64)]
    return [("all-zero", [0] * 64, 0), ("alternating-cancellation", alt, 32),
            ("signed-ramp", ramp, -32), ("sparse-positive", sparse, 1155)]


def _atomic_vectors():  # examples/workgroup_sync_v1/src/vectors.rs:72-109
    ramp = list(range(64))
    return [("none-eligible", 17, ramp, [0] * 64, 17),
            ("all-eligible", 0, ramp, [1] * 64, 2016),
            ("alternating-eligible", 11, ramp, [int(lane % 2 == 0) for lane in range(64)], 1003),
            ("sparse-eligible", 1000, ramp, [int(lane % 13 == 0) for lane in range(64)], 1130)]


@pytest.mark.parametrize("name,values,expected", _reduction_vectors())
def test_lds_reduction_vectors(name, values, expected):
    assert O.lds_reduce_i32(values) == (O.OK, expected)


def test_lds_reduction_rejects_out_of_range_sum():
    assert O.lds_reduce_i32([2**26] * 64)[0] == O.ERR_OVERFLOW
    assert O.lds_reduce_i32([-(2**31)] + [-1] + [0] * 62)[0] == O.ERR_OVERFLOW
    assert O.lds_reduce_i32([2**31 - 1] + [0] * 63) == (O.OK, 2**31 - 1)


@pytest.mark.parametrize("name,initial,values,eligible,expected", _atomic_vectors())
def test_atomic_vectors(name, initial, values, eligible, expected):
    assert O.atomic_add_u32(initial, values, eligible) == (O.OK, expected)


def test_atomic_rejects_overflow():
    assert O.atomic_add_u32(2**32 - 1, [1] * 64, [1] + [0] * 63)[0] == O.ERR_OVERFLOW


# ---- routing output consistency ---------------------------------------------------------

def candidate(pairs, tokens=8, experts=4, capacity=4):
    """The reference's canonical routing for given top-2 pairs
    (moe_routing_expert_bridge_v1.rs:628-670), produced by the oracle router
    from logits that rank the pair first and second."""
    logits = np.zeros((tokens, experts), np.float32)
    for t, (a, b) in enumerate(pairs):
        logits[t, a], logits[t, b] = 2.0, 1.0
    rc, outs = O.moe_top2_route(logits, tokens, experts, capacity)
    assert rc == O.OK
    assert [tuple(outs["top2_experts"][2 * t:2 * t + 2]) for t in range(tokens)] == list(pairs)
    return outs


def repeated(first, second):
    return candidate([(first, second)] * 8)


def check(outs, tokens=8, experts=4, capacity=4):
    return O.moe_routing_check(outs, tokens, experts, capacity)


def test_repeated_base_is_consistent():
    base = repeated(0, 1)
    assert list(base["requested_counts"]) == [8, 8, 0, 0]
    assert list(base["expert_offsets"]) == [0, 4, 8, 8, 8]
    assert check(base)[0] == "ok"


def _mutated(base, key, index, value=None, delta=None):
    m = {k: v.copy() for k, v in base.items()}
    m[key][index] = value if value is not None else int(m[key][index]) + delta
    return m


def test_hostile_mutations_fail_at_named_relations():
    """moe_routing_expert_bridge_v1.rs:738-851, including the four exact
    error values the reference asserts."""
    b = repeated(0, 1)
    assert check(_mutated(b, "expert_offsets", 2, delta=-1))[0] == "offset_mismatch"
    assert check(_mutated(b, "admitted_counts", 0, delta=-1))[0] == "admitted_count"
    assert check(_mutated(b, "requested_counts", 0, delta=-1))[0] == "requested_count"
    assert check(_mutated(b, "admitted_counts", 0, 5)) == ("capacity", 0, 0, 5)
    kind, index, _, _ = check(_mutated(b, "expert_offsets", 2, 3))
    assert (kind, index) == ("nonmonotone_offsets", 1)
    assert check(_mutated(b, "route_slots", 1, int(b["route_slots"][0])))[0] == "duplicate_slot"
    assert check(_mutated(b, "route_slots", 0, 16))[0] == "slot_out_of_range"
    assert check(_mutated(b, "permutation", 0, 2))[0] == "permutation"
    assert check(_mutated(b, "inverse", 0, 1))[0] == "inverse"
    assert check(_mutated(b, "route_slots", 8, 0)) == ("duplicate_slot", 8, 0, 0)
    assert check(_mutated(b, "inverse", 8, 0)) == ("inverse", 8, O.DROP_ROUTE, 0)
    assert check(_mutated(b, "permutation", 8, 0)) == ("permutation_tail", 8, 0, 0)


def test_cross_snapshot_substitution_is_rejected():
    """moe_routing_expert_bridge_v1.rs:853-874."""
    first, second, reversed_ = repeated(0, 1), repeated(2, 3), repeated(1, 0)
    sub = {k: v.copy() for k, v in first.items()}
    sub["admitted_counts"] = second["admitted_counts"].copy()
    sub["expert_offsets"] = second["expert_offsets"].copy()
    assert check(sub)[0] == "admitted_count"
    sub = {k: v.copy() for k, v in first.items()}
    sub["inverse"] = reversed_["inverse"].copy()
    assert check(sub)[0] == "inverse"


def test_every_router_output_is_consistent():
    """The reference's differential witness (bridge tests :683-718): routings
    the router produces are all accepted -- over random logits, token counts,
    expert counts and capacities."""
    rng = np.random.default_rng(3)
    for tokens, experts, capacity in [(8, 4, 4), (64, 8, 20), (333, 5, 0xFFFFFFFF), (512, 16, 3),
                                      (1, 2, 1), (100, 64, 7)]:
        rc, outs = O.moe_top2_route(rng.standard_normal((tokens, experts)).astype(np.float32),
                                    tokens, experts, capacity)
        assert rc == O.OK
        assert check(outs, tokens, experts, capacity)[0] == "ok"


def test_out_of_range_and_duplicate_experts():
    b = repeated(0, 1)
    assert check(_mutated(b, "top2_experts", 5, 4)) == ("expert_out_of_range", 5, 0, 4)
    assert check(_mutated(b, "top2_experts", 5, 0)) == ("duplicate_token_expert", 2, 0, 0)
    # the earlier token's violation wins over a later one
    m = _mutated(b, "top2_experts", 9, 9)
    m["top2_experts"][2] = 1
    assert check(m) == ("duplicate_token_expert", 1, 0, 1)
