"""Pins the MoE router / expert oracles (examples/moe_top2_v1/tests/oracle.rs,
examples/moe_expert_v1/tests/pipeline_oracle.rs) and the OCP e4m3 oracle
(closed forms of the OCP OFP8 specification)."""
import math

import numpy as np
import pytest

from golden import reference_vectors as rv

DROP = 0xFFFFFFFF


def route(oracle, logits, tokens=8, experts=4, capacity=4):
    rc, out = oracle.moe_top2_route(np.array(logits, np.float32), tokens, experts, capacity)
    assert rc == 0
    return out


def test_routing_pins(oracle):
    nominal = route(oracle, rv.MOE_VECTORS["nominal-balanced"])
    pin = rv.MOE_PINS["nominal-balanced"]
    for key in ("requested_counts", "admitted_counts", "expert_offsets"):
        assert nominal[key].tolist() == pin[key]
    assert DROP not in nominal["route_slots"] and DROP not in nominal["permutation"]

    eq = route(oracle, rv.MOE_VECTORS["all-equal-tie-break-and-empty-experts"])
    pin = rv.MOE_PINS["all-equal-tie-break-and-empty-experts"]
    assert all(list(eq["top2_experts"][2 * t:2 * t + 2]) == pin["top2_pairs"] for t in range(8))
    for key in ("requested_counts", "admitted_counts", "expert_offsets"):
        assert eq[key].tolist() == pin[key]
    assert np.all(eq["permutation"][8:] == DROP)

    ov = route(oracle, rv.MOE_VECTORS["stable-capacity-overflow"])
    pin = rv.MOE_PINS["stable-capacity-overflow"]
    assert ov["requested_counts"][0] == pin["requested0"]
    off = ov["expert_offsets"]
    assert ov["permutation"][off[0]:off[1]].tolist() == pin["expert0_routes"]
    for r in pin["dropped_routes"]:
        assert ov["route_slots"][r] == DROP and ov["inverse"][r] == DROP

    em = route(oracle, rv.MOE_VECTORS["empty-experts"])
    assert em["requested_counts"].tolist() == rv.MOE_PINS["empty-experts"]["requested_counts"]
    assert em["expert_offsets"][2] == em["expert_offsets"][3] == em["expert_offsets"][4]


def test_permutation_inverse_round_trip_and_determinism(oracle):
    for name, logits in rv.MOE_VECTORS.items():
        out = route(oracle, logits)
        again = route(oracle, logits)
        assert all(np.array_equal(out[k], again[k]) for k in out)
        accepted = int(out["expert_offsets"][4])
        for slot in range(accepted):
            r = int(out["permutation"][slot])
            assert r < 16 and out["route_slots"][r] == slot and out["inverse"][r] == slot, name
        assert np.all(out["permutation"][accepted:] == DROP)


def test_adversarial_signed_zero_ties(oracle):
    out = route(oracle, rv.MOE_VECTORS["adversarial-finite-values"])
    # token 3 = [MIN, -0.0, +0.0, MIN_POSITIVE]: -0 == +0 ties to the lower id
    assert out["top2_experts"][6:8].tolist() == [3, 1]
    # token 5 = [-42, -42, -42, -43]
    assert out["top2_experts"][10:12].tolist() == [0, 1]


def test_nonfinite_and_wrong_length_fail_closed(oracle):
    for bad in (np.nan, np.inf, -np.inf):
        lg = np.zeros(32, np.float32)
        lg[11] = bad
        rc, out = oracle.moe_top2_route(lg, 8, 4, 4, fill=0x76543210)
        assert rc == oracle.ERR_NONFINITE
        assert all(np.all(v == 0x76543210) for v in out.values())


def test_sort_selector_equals_running_selector_brute_force(oracle):
    """The reference's two independent selectors (oracle.rs:63-82 sort and
    kernel.rs:25-59 running max) agree on every tie-heavy small input."""
    rng = np.random.default_rng(1)
    for experts in (2, 3, 4, 8):
        for _ in range(400):
            logits = rng.integers(-2, 3, size=(16, experts)).astype(np.float32)
            logits[rng.random(logits.shape) < 0.1] = -0.0
            rc, out = oracle.moe_top2_route(logits, 16, experts, 0xFFFFFFFF)
            for t in range(16):
                run = oracle.moe_select_top2_running(logits[t])
                assert out["top2_experts"][2 * t:2 * t + 2].tolist() == run.tolist()
                # closed form: stable argsort by (-score, id)
                order = sorted(range(experts), key=lambda e: (-float(logits[t, e]), e))
                assert run.tolist() == order[:2]


def test_large_router_scan_invariants(oracle):
    rng = np.random.default_rng(2)
    T, E = 4096, 8
    logits = oracle.bf16_to_f32(oracle.bf16_from_f32(rng.standard_normal(T * E).astype(np.float32)))
    for cap in (0xFFFFFFFF, 600, 1024):
        rc, out = oracle.moe_top2_route(logits, T, E, cap)
        assert rc == 0
        req = np.bincount(out["top2_experts"], minlength=E)
        assert np.array_equal(out["requested_counts"], req)
        assert np.array_equal(out["admitted_counts"], np.minimum(req, cap))
        assert np.array_equal(out["expert_offsets"], np.concatenate([[0], np.cumsum(np.minimum(req, cap))]))
        t2 = out["top2_experts"].reshape(T, 2)
        assert np.all(t2[:, 0] != t2[:, 1])
    w = oracle.moe_top2_weights(logits, T, E, out["top2_experts"])
    pairs = w.reshape(T, 2)
    assert np.all(pairs[:, 0] + pairs[:, 1] == np.float32(1.0))
    assert np.all(pairs[:, 0] >= 0.5)
    l0 = logits.reshape(T, E)[np.arange(T), t2[:, 0]].astype(np.float64)
    l1 = logits.reshape(T, E)[np.arange(T), t2[:, 1]].astype(np.float64)
    assert np.allclose(pairs[:, 0], 1 / (1 + np.exp(l1 - l0)), atol=1e-6)


def _expert_inputs(oracle, logits):
    acts = rv.moe_expert_activations(oracle.bf16_from_f32)
    weights = rv.moe_expert_weights(oracle.bf16_from_f32)
    rw = rv.moe_expert_route_weights()
    routing = route(oracle, logits)
    return acts, weights, rw, routing


@pytest.mark.parametrize("logits_fn", [rv.moe_expert_equal_logits, rv.moe_expert_balanced_logits])
def test_expert_pipeline_equals_independent_oracle(oracle, logits_fn):
    logits = np.array(logits_fn(), np.float32)
    acts, weights, rw, routing = _expert_inputs(oracle, logits)
    rc1, pipe = oracle.moe_expert_pipeline_v1(logits, acts, weights, rw, routing)
    rc2, ind = oracle.moe_expert_independent_v1(logits, acts, weights, rw, routing)
    assert rc1 == 0 and rc2 == 0
    for key in ("expert_output_tiles", "compact_output", "combined_output"):
        assert np.array_equal(pipe[key].view(np.uint32), ind[key].view(np.uint32)), key
    for e in range(4):
        active = int(routing["admitted_counts"][e])
        assert np.all(pipe["activation_tiles"][e * 256 + active * 16:(e + 1) * 256] == 0)
        assert np.all(pipe["expert_output_tiles"][e * 256 + active * 16:(e + 1) * 256] == 0)
    for r in range(16):
        slot = routing["inverse"][r]
        if slot == DROP:
            assert np.all(ind["route_output"][r * 16:(r + 1) * 16] == 0)
        else:
            assert np.array_equal(ind["route_output"][r * 16:(r + 1) * 16],
                                  pipe["compact_output"][slot * 16:(slot + 1) * 16])


def test_expert_weight_policy_fails_closed(oracle):
    logits = np.array(rv.moe_expert_balanced_logits(), np.float32)
    acts, weights, rw, routing = _expert_inputs(oracle, logits)
    bad = rw.copy()
    bad[3] = np.float32(0.3)
    assert oracle.moe_expert_independent_v1(logits, acts, weights, bad, routing)[0] == \
        oracle.ERR_WEIGHTS
    a2 = acts.copy()
    a2[5] = 0x7F80
    assert oracle.moe_expert_independent_v1(logits, a2, weights, rw, routing)[0] == \
        oracle.ERR_NONFINITE


def test_ffn_route_closed_form(oracle):
    rng = np.random.default_rng(4)
    h, f = 32, 48
    x = oracle.bf16_from_f32(rng.standard_normal(h).astype(np.float32))
    wg = oracle.bf16_from_f32((rng.standard_normal(f * h) * 0.2).astype(np.float32))
    wu = oracle.bf16_from_f32((rng.standard_normal(f * h) * 0.2).astype(np.float32))
    wd = oracle.bf16_from_f32((rng.standard_normal(h * f) * 0.2).astype(np.float32))
    hidden, y = oracle.moe_ffn_route(x, wg, wu, wd, h, f)
    xf = oracle.bf16_to_f32(x).astype(np.float64)
    g = oracle.bf16_to_f32(wg).reshape(f, h).astype(np.float64) @ xf
    u = oracle.bf16_to_f32(wu).reshape(f, h).astype(np.float64) @ xf
    hid = g / (1 + np.exp(-g)) * u
    assert np.allclose(oracle.bf16_to_f32(hidden), hid, rtol=1e-2, atol=1e-3)
    yy = oracle.bf16_to_f32(wd).reshape(h, f).astype(np.float64) @ oracle.bf16_to_f32(hidden)
    assert np.allclose(y, yy, rtol=1e-5, atol=1e-5)


# ---- OCP e4m3 ---------------------------------------------------------------

def test_e4m3_decode_table_closed_form(oracle):
    table = oracle.fp8_decode_table()
    for b in range(256):
        s, e, m = b >> 7, (b >> 3) & 15, b & 7
        if e == 15 and m == 7:
            assert math.isnan(table[b])
            continue
        val = m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
        assert table[b] == (-val if s else val)
    assert table[0x7E] == 448.0 and table[0x01] == 2.0 ** -9 and table[0x08] == 2.0 ** -6


def test_e4m3_encode_is_rne_with_saturation(oracle):
    table = oracle.fp8_decode_table()
    finite = [b for b in range(256) if not math.isnan(table[b])]
    for b in finite:  # exact values round-trip (sign of zero kept)
        assert oracle.fp8_from_f32(float(table[b])) == b
    # brute force against nearest-even over the positive finite set
    pos = sorted((float(table[b]), b) for b in range(0x7F))
    rng = np.random.default_rng(9)
    xs = np.concatenate([rng.uniform(0, 460, 20000), rng.uniform(0, 0.02, 5000),
                         [(pos[i][0] + pos[i + 1][0]) / 2 for i in range(len(pos) - 1)]])
    for x in xs.astype(np.float32):
        x = float(x)
        got = oracle.fp8_from_f32(x)
        if x >= 448.0:
            assert got == 0x7E
            continue
        best = min(pos, key=lambda p: (abs(p[0] - x), p[1] & 1))
        assert table[got] == best[0], x
        assert oracle.fp8_from_f32(-x) == (got | 0x80)
    assert oracle.fp8_from_f32(1e9) == 0x7E and oracle.fp8_from_f32(-1e9) == 0xFE
    assert oracle.fp8_from_f32(float("nan")) & 0x7F == 0x7F


def test_fp8_gemm_points_closed_form(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(64 * 256).astype(np.float32)
    y = rng.standard_normal(32 * 256).astype(np.float32)
    sa = np.float32(oracle.amax_f32(x)) / np.float32(448.0)
    sb = np.float32(oracle.amax_f32(y)) / np.float32(448.0)
    assert oracle.amax_f32(x) == np.abs(x).max()
    qa = oracle.quantize_e4m3(x, sa).reshape(64, 256)
    qb = oracle.quantize_e4m3(y, sb).reshape(32, 256)
    table = oracle.fp8_decode_table().astype(np.float64)
    assert np.abs(table[qa.ravel()] * sa - x).max() <= 0.0625 * float(np.abs(x).max()) / 448 * 448
    ii = np.repeat(np.arange(64), 32)
    jj = np.tile(np.arange(32), 64)
    of, ob = oracle.gemm_fp8_points(256, qa[ii], qb[jj], float(sa * sb))
    exact = (table[qa] @ table[qb].T)[ii, jj] * float(sa * sb)
    assert np.allclose(of, exact, rtol=1e-5, atol=1e-4)
    assert np.array_equal(ob, oracle.bf16_from_f32(of))


def test_fp8_rows_equal_points_form(oracle):
    """The row-block fp8 GEMM oracle (used for whole-row parity at config 4)
    equals the per-point form bit for bit, on a tail column block too."""
    rng = np.random.default_rng(1)
    m, n, k = 5, 37, 300
    a = rng.integers(0, 256, m * k).astype(np.uint8)
    b = rng.integers(0, 256, n * k).astype(np.uint8)
    a[(a & 0x7F) == 0x7F] = 0  # no NaN encodings
    b[(b & 0x7F) == 0x7F] = 0
    rows = oracle.gemm_fp8_nt_rows(n, k, a, b, 0.37, 1, 4)
    ii, jj = np.meshgrid(np.arange(1, 4), np.arange(n), indexing="ij")
    of, _ = oracle.gemm_fp8_points(k, a.reshape(m, k)[ii.ravel()], b.reshape(n, k)[jj.ravel()],
                                   0.37)
    assert rows.ravel().view(np.uint32).tolist() == of.view(np.uint32).tolist()


def test_moe_ffn_routes_equal_single_route(oracle):
    """The OpenMP batch of expert FFN routes equals the single-route form
    bit for bit, and the single-route form equals a float64 evaluation of
    silu(x Wg^T) * (x Wu^T) then Wd within the bf16 rounding of the hidden
    activation."""
    rng = np.random.default_rng(2)
    tokens, h, f, e = 6, 64, 40, 3
    x = oracle.bf16_from_f32(rng.standard_normal(tokens * h)).reshape(tokens, h)
    wg, wu, wd = (oracle.bf16_from_f32(rng.standard_normal(e * f * h) * 0.1) for _ in range(3))
    tok = np.array([0, 5, 2, 2, 4], np.uint32)
    exp_ = np.array([1, 0, 2, 1, 2], np.uint32)
    y = oracle.moe_ffn_routes(x, wg, wu, wd, h, f, tok, exp_)
    for r, (t, ex) in enumerate(zip(tok, exp_)):
        sl = slice(int(ex) * f * h, (int(ex) + 1) * f * h)
        hid, y1 = oracle.moe_ffn_route(x[t], wg[sl], wu[sl], wd[sl], h, f)
        assert y[r].view(np.uint32).tolist() == y1.view(np.uint32).tolist()
        xf = oracle.bf16_to_f32(x[t]).astype(np.float64)
        g = oracle.bf16_to_f32(wg[sl]).reshape(f, h).astype(np.float64) @ xf
        u = oracle.bf16_to_f32(wu[sl]).reshape(f, h).astype(np.float64) @ xf
        hv = g / (1.0 + np.exp(-g)) * u
        assert np.max(np.abs(oracle.bf16_to_f32(hid) - hv)) <= 2.0 ** -7 * np.max(np.abs(hv))
        ref = oracle.bf16_to_f32(wd[sl]).reshape(h, f).astype(np.float64) @ oracle.bf16_to_f32(hid)
        assert np.max(np.abs(y1 - ref)) <= 1e-5 * np.max(np.abs(ref))
