"""Pins the flash-attention and row-softmax oracle restatements against the
reference's tests (examples/flash_attention_v1/tests/oracle.rs,
examples/row_softmax_v1/tests/numerical_contract.rs) and closed forms."""
import math

import numpy as np

from golden import reference_vectors as rv


def _vec(name):
    for v in rv.flash_vectors_v1():
        if v[0] == name:
            return v
    raise KeyError(name)


def test_flash_corpus_is_finite_with_bounded_denominators(oracle):
    names = [v[0] for v in rv.flash_vectors_v1()]
    assert names == ["nominal-mixed-sign", "all-equal-logits", "latest-causal-key-dominates",
                     "causal-mask-weight-probe"]
    for name, q, k, v in rv.flash_vectors_v1():
        rc, out, mx, den = oracle.flash_attention_v1(q, k, v)
        assert rc == 0, name
        assert np.all(np.isfinite(out)) and np.all(np.isfinite(mx))
        assert np.all((den >= 1.0) & (den <= 8.0))


def test_flash_all_equal_logits_give_exact_prefix_means(oracle):
    _, q, k, v = _vec("all-equal-logits")
    rc, out, _, _ = oracle.flash_attention_v1(q, k, v)
    for r in range(8):
        for c in range(16):
            exp = sum(float(v[j * 16 + c]) for j in range(r + 1)) / (r + 1)
            assert out[r * 16 + c] == np.float32(exp)


def test_flash_dominant_key_selects_latest_value(oracle):
    _, q, k, v = _vec("latest-causal-key-dominates")
    rc, out, _, _ = oracle.flash_attention_v1(q, k, v)
    assert np.all(np.abs(out - v) <= 1e-5)


def test_flash_future_keys_are_masked(oracle):
    _, q, k, v = _vec("nominal-mixed-sign")
    _, base, _, _ = oracle.flash_attention_v1(q, k, v)
    for first in range(1, 8):
        k2, v2 = k.copy(), v.copy()
        k2[first * 16:] += np.float32(1000.0)
        v2[first * 16:] += np.float32(1000.0)
        _, obs, _, _ = oracle.flash_attention_v1(q, k2, v2)
        assert np.array_equal(obs[:first * 16].view(np.uint32), base[:first * 16].view(np.uint32))


def test_flash_probe_row_sums_and_zero_future_weight(oracle):
    _, q, k, v = _vec("causal-mask-weight-probe")
    _, out, _, _ = oracle.flash_attention_v1(q, k, v)
    for r in range(8):
        row = out[r * 16:(r + 1) * 16]
        assert abs(float(np.sum(row[:8], dtype=np.float32)) - 1.0) <= 2e-7
        assert np.all(row[r + 1:8] == 0.0) and np.all(row[8:] == 0.0)


def test_flash_fail_closed_without_output_writes(oracle):
    _, q, k, v = _vec("nominal-mixed-sign")
    L = oracle.lib()
    out = np.full(128, 123.5, np.float32)
    assert L.fe2o3o_flash_attention_v1(q.ctypes.data, 127, k.ctypes.data, 128, v.ctypes.data,
                                       128, out.ctypes.data, 128, None, None) == oracle.ERR_LENGTH
    assert np.all(out == 123.5)
    for which, bad in ((0, np.nan), (1, np.inf), (2, -np.inf)):
        t = [q.copy(), k.copy(), v.copy()]
        t[which][37] = bad
        rc, o, _, _ = oracle.flash_attention_v1(*t)
        assert rc == oracle.ERR_NONFINITE and np.all(np.isnan(o))
    _, q2, k2, v2 = _vec("all-equal-logits")
    q2 = q2.copy()
    q2[0] = np.finfo(np.float32).max
    k2 = k2.copy()
    k2[0] = 2.0
    rc, o, _, _ = oracle.flash_attention_v1(q2, k2, v2)
    assert rc == oracle.ERR_INTERMEDIATE and np.all(np.isnan(o))


def test_general_flash_rows_match_fixed_profile(oracle):
    """The [B,H,S,D] form reproduces the fixed causal profile when fed the
    same (bf16-exact) data, and its non-causal mode is invariant to a key
    permutation (closed form of a sum)."""
    for name, q, k, v in rv.flash_vectors_v1():
        if name == "nominal-mixed-sign":
            continue  # not bf16-exact
        qb, kb, vb = (oracle.bf16_from_f32(t) for t in (q, k, v))
        assert np.array_equal(oracle.bf16_to_f32(qb), q)
        rc, out, lse = oracle.flash_attention_rows_bf16(qb, kb, vb, 8, 16, True, 0.25,
                                                        np.zeros(8, np.uint32),
                                                        np.arange(8, dtype=np.uint32))
        rc2, ref, mx, den = oracle.flash_attention_v1(q, k, v)
        assert rc == 0 and rc2 == 0
        assert np.array_equal(out.ravel().view(np.uint32), ref.view(np.uint32)), name
        assert np.allclose(lse, mx + np.log(den), rtol=0, atol=1e-6)
    rng = np.random.default_rng(0)
    s, d = 64, 32
    q = oracle.bf16_from_f32(rng.standard_normal(s * d).astype(np.float32))
    k = oracle.bf16_from_f32(rng.standard_normal(s * d).astype(np.float32))
    v = oracle.bf16_from_f32(rng.standard_normal(s * d).astype(np.float32))
    perm = rng.permutation(s)
    kp = k.reshape(s, d)[perm].ravel()
    vp = v.reshape(s, d)[perm].ravel()
    rows = np.arange(s, dtype=np.uint32)
    bh = np.zeros(s, np.uint32)
    _, o1, l1 = oracle.flash_attention_rows_bf16(q, k, v, s, d, False, 0.125, bh, rows)
    _, o2, l2 = oracle.flash_attention_rows_bf16(q, kp, vp, s, d, False, 0.125, bh, rows)
    assert np.allclose(o1, o2, atol=1e-6) and np.allclose(l1, l2, atol=1e-6)
    # brute-force closed form in numpy f64
    qf = oracle.bf16_to_f32(q).reshape(s, d).astype(np.float64)
    kf = oracle.bf16_to_f32(k).reshape(s, d).astype(np.float64)
    vf = oracle.bf16_to_f32(v).reshape(s, d).astype(np.float64)
    sc = qf @ kf.T * 0.125
    sc = np.where(np.tril(np.ones((s, s), bool)), sc, -np.inf)
    p = np.exp(sc - sc.max(1, keepdims=True))
    ref = (p @ vf) / p.sum(1, keepdims=True)
    _, oc, lc = oracle.flash_attention_rows_bf16(q, k, v, s, d, True, 0.125, bh, rows)
    assert np.allclose(oc, ref, atol=1e-6)
    assert np.allclose(lc, sc.max(1) + np.log(p.sum(1)), atol=1e-5)


# ---- row softmax -------------------------------------------------------------

def test_softmax_rejections_leave_output_untouched(oracle):
    L = oracle.lib()
    out = np.full(4, 19.0, np.float32)
    z3 = np.zeros(3, np.float32)
    assert oracle.row_softmax_oracle_v1(np.zeros(0, np.float32))[0] == oracle.ERR_EMPTY
    assert oracle.row_softmax_oracle_v1(np.zeros(4, np.float32),
                                        mask=np.zeros(4, np.uint8), out=out)[0] == \
        oracle.ERR_NO_ACTIVE
    for idx, bad in ((0, np.nan), (1, np.inf), (3, -np.inf)):
        x = np.zeros(4, np.float32)
        x[idx] = bad
        assert oracle.row_softmax_oracle_v1(x, mask=np.array([1, 0, 1, 1], np.uint8),
                                            out=out)[0] == oracle.ERR_NONFINITE
    assert np.all(out == 19.0)
    big = np.zeros(4097, np.float32)
    o2 = np.full(4097, 7.0, np.float32)
    assert oracle.row_softmax_oracle_v1(big, out=o2)[0] == oracle.ERR_TOO_LARGE
    assert np.all(o2 == 7.0)
    del L, z3


def test_softmax_mask_signed_zero_subnormal_underflow(oracle):
    x = np.array([-0.0, 0.0, rv.bits_f32(1), -200.0], np.float32)
    mask = np.array([1, 0, 1, 1], np.uint8)
    rc, out, st = oracle.row_softmax_oracle_v1(x, mask=mask)
    assert rc == 0 and st["active"] == 3
    assert np.float32(st["maximum"]).view(np.uint32) == 1
    assert out.view(np.uint32)[1] == 0 and out[3] == 0.0 and out[0] > 0 and out[2] > 0
    assert oracle.compare_row_softmax_v1(out, out, mask)[0] == 0


def test_softmax_corpus_and_equal_row_bits(oracle):
    for row in rv.softmax_corpus_v1():
        rc, out, st = oracle.row_softmax_oracle_v1(row)
        assert rc == 0 and np.isfinite(st["maximum"]) and st["denominator"] >= 1.0
        assert oracle.compare_row_softmax_v1(out, out)[0] == 0
    rc, out, _ = oracle.row_softmax_oracle_v1(np.zeros(64, np.float32))
    assert np.all(out.view(np.uint32) == np.float32(1.0 / 64.0).view(np.uint32))


def test_softmax_comparison_rejects_substitutions(oracle):
    x = np.array([0.0, 1.0, 2.0, 3.0], np.float32)
    mask = np.array([1, 0, 1, 1], np.uint8)
    _, exp, _ = oracle.row_softmax_oracle_v1(x, mask=mask)
    wrong = exp.copy()
    wrong[2] += np.float32(0.01)
    assert oracle.compare_row_softmax_v1(exp, wrong, mask) == (oracle.ERR_MISMATCH, 2)
    sub = exp.copy()
    sub[0] += np.float32(0.01)
    assert oracle.compare_row_softmax_v1(sub, exp, mask) == (oracle.ERR_MISMATCH, 0)
    wm = exp.copy()
    wm[1] = -0.0
    assert oracle.compare_row_softmax_v1(exp, wm, mask) == (oracle.ERR_MISMATCH, 1)
    assert oracle.compare_row_softmax_v1(exp, exp, mask, abs_tol=float("nan"))[0] == \
        oracle.ERR_POLICY
    nf = exp.copy()
    nf[0] = np.nan
    assert oracle.compare_row_softmax_v1(exp, nf, mask)[0] == oracle.ERR_NONFINITE
    ws = exp * np.float32(0.99)
    ws[1] = 0.0
    assert oracle.compare_row_softmax_v1(exp, ws, mask, abs_tol=1.0, rel_tol=1.0,
                                         max_ulps=2**32 - 1)[0] == oracle.ERR_SUM


def test_softmax_f32_reference_matches_f64_oracle_within_policy(oracle):
    cases = rv.softmax_production_cases_v1()
    for name in ("normal", "equal", "dominant"):
        rc, ref32 = oracle.row_softmax_reference_v1(cases[name])
        rc2, ref64, _ = oracle.row_softmax_oracle_v1(cases[name])
        assert rc == 0 and rc2 == 0
        assert oracle.compare_row_softmax_v1(ref64, ref32)[0] == 0, name
    assert oracle.row_softmax_reference_v1(cases["exceptional"])[0] == oracle.ERR_NONFINITE
    # closed form for the dominant row: p37 = 1/(1+63 e^-64)
    _, out, _ = oracle.row_softmax_oracle_v1(cases["dominant"])
    assert out[37] == np.float32(1.0 / (1.0 + 63.0 * math.exp(-64.0)))


def test_softmax_rows_is_rowwise_oracle(oracle):
    x = oracle.fill_normal_f32(8 * 4096, 3, 1, 1.0)
    rc, out = oracle.row_softmax_rows(x, 8, 4096, threads=4)
    assert rc == 0
    for r in range(8):
        _, one, _ = oracle.row_softmax_oracle_v1(x[r * 4096:(r + 1) * 4096])
        assert np.array_equal(out[r].view(np.uint32), one.view(np.uint32))


def test_row_softmax_check_rows_counts_what_the_row_compare_rejects(oracle):
    """The many-row check (fe2o3o_row_softmax_check_rows, used on config 3c's
    million rows) is the per-row oracle plus the contract's comparison: it
    passes the oracle's own output, and on planted mistakes (on the CPU) it
    fails exactly the rows that compare_row_softmax_v1 rejects, reporting the
    first one, a NaN as a NaN difference and the row-sum error."""
    rng = np.random.default_rng(11)
    rows, cols = 257, 4096
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    rc, ref = oracle.row_softmax_rows(x, rows, cols)
    assert rc == 0
    rc, st = oracle.row_softmax_check_rows(x, ref, rows, cols)
    assert rc == 0 and st["failing_rows"] == 0 and st["first_failing_row"] == rows
    assert st["max_abs_diff"] == 0.0 and st["max_row_sum_err"] < 1e-6
    y = ref.copy()
    y[200, 5] += 1e-4        # beyond abs 3e-6 + rel 3e-5 and 64 ULP
    y[31, 4000] *= 1.5
    y[100, 0] *= 1.0 + 1e-6  # within the policy
    rc, st = oracle.row_softmax_check_rows(x, y, rows, cols)
    assert rc == 0 and st["failing_rows"] == 2 and st["first_failing_row"] == 31
    want = [r for r in range(rows)
            if oracle.compare_row_softmax_v1(ref[r], y[r], **oracle.GFX_SOFTMAX_POLICY)[0] != 0]
    assert want == [31, 200]
    assert abs(st["max_abs_diff"] - float(np.max(np.abs(y.astype(np.float64) - ref)))) < 1e-12
    y[7, 7] = np.nan
    rc, st = oracle.row_softmax_check_rows(x, y, rows, cols)
    assert st["failing_rows"] == 3 and st["first_failing_row"] == 7
    assert np.isnan(st["max_abs_diff"]) and np.isnan(st["max_row_sum_err"])
