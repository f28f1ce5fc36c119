"""Pins the GEMM oracle restatement against the reference's own golden vectors
(examples/tiled_gemm_v1/tests/*, examples/scalar_gemm_v1/src/harness.rs,
examples/tiled_gemm_general_v1/hardware-harness) and against closed forms."""
import struct
from fractions import Fraction

import numpy as np
import pytest

from golden import reference_vectors as rv


def f32bits(arr):
    return [int(x) for x in np.asarray(arr, np.float32).view(np.uint32)]


# ---- bf16 vocabulary ---------------------------------------------------------

def test_bf16_widening_is_exact_for_every_encoding(oracle):
    bits = np.arange(65536, dtype=np.uint32)
    widened = oracle.bf16_to_f32(bits.astype(np.uint16)).view(np.uint32)
    assert np.array_equal(widened, bits << 16)
    # numerical_contract.rs:113-121
    assert oracle.lib().fe2o3o_bf16_to_f32(0x8000) == 0.0
    assert struct.pack("<f", oracle.lib().fe2o3o_bf16_to_f32(0x8000)) == b"\x00\x00\x00\x80"
    assert oracle.lib().fe2o3o_bf16_to_f32(0x3F80) == 1.0


def test_bf16_narrowing_rne_closed_form(oracle):
    # half.rs:182-190: ties to even, NaN quieted, round trip of every finite
    # encoding.
    L = oracle.lib()
    every = np.arange(65536, dtype=np.uint16)
    finite = every[(every & 0x7F80) != 0x7F80]
    back = oracle.bf16_from_f32(oracle.bf16_to_f32(finite))
    assert np.array_equal(back, finite)
    assert L.fe2o3o_bf16_from_f32(rv.bits_f32(0x3F808000)) == 0x3F80  # tie -> even
    assert L.fe2o3o_bf16_from_f32(rv.bits_f32(0x3F818000)) == 0x3F82  # tie -> even (up)
    assert L.fe2o3o_bf16_from_f32(rv.bits_f32(0x3F808001)) == 0x3F81
    assert L.fe2o3o_bf16_from_f32(rv.bits_f32(0x7F800001)) == 0x7FC0  # quiet NaN
    assert L.fe2o3o_bf16_from_f32(rv.bits_f32(0x7F7FFFFF)) == 0x7F80  # overflow to inf


# ---- reference generator (inputs.rs) ------------------------------------------

def test_generator_v1_bytes_are_pinned(oracle):
    pin = rv.GENERATOR_PIN
    m, n, k = pin["shape"]
    a, b = oracle.generate_inputs_v1(m, n, k, pin["seed"])
    assert a.tolist() == pin["a_bits"]
    assert b.tolist() == pin["b_bits"]
    rc, _, _ = oracle.validate_evidence_inputs_v1(m, n, k, a, b)
    assert rc == 0
    rc, out = oracle.tiled_gemm_arithmetic_v1(m, n, k, a, b)
    assert rc == 0 and f32bits(out) == pin["out_bits"]


def test_generator_determinism_separation_and_alphabet(oracle):
    a1, b1 = oracle.generate_inputs_v1(16, 16, 16, 0x123456789ABCDEF0)
    a2, b2 = oracle.generate_inputs_v1(16, 16, 16, 0x123456789ABCDEF0)
    assert np.array_equal(a1, a2) and np.array_equal(b1, b2)
    assert not np.array_equal(a1, b1)
    a3, b3 = oracle.generate_inputs_v1(16, 16, 16, 0x123456789ABCDEF1)
    assert not np.array_equal(a1, a3) and not np.array_equal(b1, b3)
    a4, _ = oracle.generate_inputs_v1(16, 32, 16, 0x1234)
    a5, _ = oracle.generate_inputs_v1(16, 16, 16, 0x1234)
    assert not np.array_equal(a4[:256], a5)
    allowed = set(rv.BF16_INPUT_PATTERN_V1)
    for mt in range(4):
        for nt in range(4):
            for kt in range(4):
                for seed in (0, 1, 2**64 - 1, 0xA5A55A5AC3C33C3C):
                    a, b = oracle.generate_inputs_v1(mt * 16, nt * 16, kt * 16, seed)
                    assert set(a.tolist()) <= allowed and set(b.tolist()) <= allowed


def test_evidence_validation_rejects_hostile_classes(oracle):
    codes = {"nan": oracle.ERR_NONFINITE, "inf": oracle.ERR_INFINITE,
             "subnormal": oracle.ERR_SUBNORMAL, "alphabet": oracle.ERR_ALPHABET}
    for bits, cls in rv.HOSTILE_BF16:
        rc, op, idx = oracle.validate_evidence_inputs_v1(1, 1, 1, np.array([bits], np.uint16),
                                                         np.array([0x3F80], np.uint16))
        assert (rc, op, idx) == (codes[cls], 0, 0), hex(bits)
    # operand and row-major index (inputs_oracle.rs:179-191)
    rc, op, idx = oracle.validate_evidence_inputs_v1(1, 2, 1, np.array([0x3F80], np.uint16),
                                                     np.array([0x3F80, 0x3F40], np.uint16))
    assert (rc, op, idx) == (oracle.ERR_ALPHABET, 1, 1)


def test_evidence_validation_admits_exactly_the_alphabet(oracle):
    allowed = set(rv.BF16_INPUT_PATTERN_V1)
    one = np.array([0x3F80], np.uint16)
    for bits in range(65536):
        rc, _, _ = oracle.validate_evidence_inputs_v1(1, 1, 1, np.array([bits], np.uint16), one)
        assert (rc == 0) == (bits in allowed), hex(bits)


def test_evidence_validation_wrong_lengths(oracle):
    a, b = oracle.generate_inputs_v1(2, 3, 2, 9)
    assert oracle.validate_evidence_inputs_v1(2, 3, 2, a[:3], b)[:2] == (oracle.ERR_LENGTH, 0)
    assert oracle.validate_evidence_inputs_v1(2, 3, 2, a, b[:5])[:2] == (oracle.ERR_LENGTH, 1)
    nan = np.array([0x7FC0], np.uint16)
    empty = np.zeros(0, np.uint16)
    assert oracle.validate_evidence_inputs_v1(0, 2**32 - 1, 2**32 - 1, nan, empty)[:2] == (
        oracle.ERR_LENGTH, 0)


# ---- arithmetic recurrence (oracle.rs:284-320) --------------------------------

def test_arithmetic_known_product_and_zero_k(oracle):
    a = oracle.bf16_from_f32([1.0, 2.0, 3.0, 4.0])
    b = oracle.bf16_from_f32([5.0, 6.0, 7.0, 8.0, 9.0, 10.0])
    rc, out = oracle.tiled_gemm_arithmetic_v1(2, 3, 2, a, b)
    assert rc == 0 and out.tolist() == [21.0, 24.0, 27.0, 47.0, 54.0, 61.0]
    for m, n in ((1, 1), (16, 16), (17, 31)):
        rc, out = oracle.tiled_gemm_arithmetic_v1(m, n, 0, np.zeros(0, np.uint16),
                                                  np.zeros(0, np.uint16))
        assert rc == 0 and all(x == 0 for x in f32bits(out))


def test_arithmetic_rounding_order_and_signed_zero(oracle):
    # inputs_oracle.rs:292-347
    one = 0x3F80
    a = np.array([one] * 3, np.uint16)
    rc, out = oracle.tiled_gemm_arithmetic_v1(1, 1, 3, a, np.array([0x4B80, one, 0xCB80], np.uint16))
    assert f32bits(out) == [0x00000000]
    rc, out = oracle.tiled_gemm_arithmetic_v1(1, 1, 3, a, np.array([0x4B80, 0xCB80, one], np.uint16))
    assert f32bits(out) == [0x3F800000]
    for a1, b1 in ((0x0000, 0xBF80), (0x8000, 0x3F80)):
        rc, out = oracle.tiled_gemm_arithmetic_v1(1, 1, 1, np.array([a1], np.uint16),
                                                  np.array([b1], np.uint16))
        assert f32bits(out) == [0]


def test_arithmetic_rejects_length_substitution(oracle):
    a, b = oracle.generate_inputs_v1(2, 3, 4, 7)
    assert oracle.tiled_gemm_arithmetic_v1(2, 3, 4, a[:-1], b)[0] == oracle.ERR_LENGTH
    assert oracle.tiled_gemm_arithmetic_v1(2, 3, 4, a, b[:-1])[0] == oracle.ERR_LENGTH
    assert oracle.tiled_gemm_arithmetic_v1(2, 3, 4, np.append(a, 0).astype(np.uint16), b)[0] == \
        oracle.ERR_LENGTH


def test_arithmetic_matches_exact_rational_sum_on_dyadic_inputs(oracle):
    # Closed form: with dyadic inputs of small magnitude every partial sum is
    # exactly representable, so the f32 recurrence equals the exact sum.
    for seed in range(4):
        m, n, k = 7, 5, 33
        a, b = oracle.generate_inputs_v1(m, n, k, seed)
        rc, out = oracle.tiled_gemm_arithmetic_v1(m, n, k, a, b)
        af = oracle.bf16_to_f32(a).reshape(m, k)
        bf = oracle.bf16_to_f32(b).reshape(k, n)
        for i in range(m):
            for j in range(n):
                exact = sum(Fraction(float(af[i, d])) * Fraction(float(bf[d, j])) for d in range(k))
                assert Fraction(float(out[i * n + j])) == exact


# ---- numerical contract (numerical_contract.rs) -------------------------------

def test_source_oracle_alpha_beta_kat(oracle):
    kat = rv.SOURCE_KAT
    m, n, k = kat["dims"]
    lda, ldb, ldc = kat["strides"]
    rc, out = oracle.evaluate_source(m, n, k, lda, ldb, ldc, kat["a"], kat["b"], kat["c"],
                                     kat["alpha"], kat["beta"])
    assert rc == 0 and f32bits(out) == kat["out_bits"]


def test_spec_extents_and_zero_k(oracle):
    kat = rv.ZERO_K_KAT
    spec, lens = kat["padded_spec"]
    assert oracle.gemm_spec_checked(*spec) == (0, lens)
    m, n, k = kat["dims"]
    rc, out = oracle.evaluate_source(m, n, k, *kat["strides"], [], [], kat["c"], kat["alpha"],
                                     kat["beta"])
    assert rc == 0 and out.tolist() == kat["out"]
    assert oracle.gemm_spec_checked(2, 3, 4, 3, 3, 3)[0] == oracle.ERR_STRIDE


def test_finite_policy_rejections(oracle):
    for bits, code in ((0x0001, oracle.ERR_SUBNORMAL), (0x8001, oracle.ERR_SUBNORMAL),
                       (0x7F80, oracle.ERR_INFINITE), (0xFF80, oracle.ERR_INFINITE),
                       (0x7FC1, oracle.ERR_NONFINITE), (0xFF81, oracle.ERR_NONFINITE)):
        rc, _ = oracle.build_hardware_expectation(1, 2, 1, 1, 2, 2, [0x3F80], [0x3F80, bits],
                                                  [0.0, 0.0], 1.0, 0.0)
        assert rc == code
    sub = rv.bits_f32(1)
    assert oracle.build_hardware_expectation(1, 1, 1, 1, 1, 1, [0x3F80], [0x3F80], [sub], 1.0,
                                             0.0)[0] == oracle.ERR_SUBNORMAL
    assert oracle.build_hardware_expectation(1, 1, 1, 1, 1, 1, [0x3F80], [0x3F80], [0.0],
                                             float("-inf"), 0.0)[0] == oracle.ERR_INFINITE
    # product overflow / subnormal intermediates (numerical_contract.rs:264-298)
    assert oracle.build_hardware_expectation(1, 1, 1, 1, 1, 1, [0x7F7F], [0x4000], [0.0], 1.0,
                                             0.0)[0] == oracle.ERR_INTERMEDIATE
    assert oracle.build_hardware_expectation(1, 1, 1, 1, 1, 1, [0x0080], [0x3F00], [0.0], 1.0,
                                             0.0)[0] == oracle.ERR_INTERMEDIATE


def test_comparison_policies(oracle):
    # numerical_contract.rs:301-380
    assert oracle.compare_hardware([0.0], [0.0], oracle.BOUNDED, -1.0, 0.0, 1)[0] == \
        oracle.ERR_POLICY
    assert oracle.compare_hardware([0.0], [0.0], oracle.BOUNDED, 0.0, 0.0, 1)[0] == \
        oracle.ERR_POLICY
    assert oracle.compare_hardware([0.0], [0.0], oracle.BOUNDED, 1.0, 0.0, 0)[0] == \
        oracle.ERR_POLICY
    rc, _ = oracle.compare_hardware([0.0], [-0.0], oracle.EXACT_BITS)
    assert rc == oracle.ERR_MISMATCH
    rc, rep = oracle.compare_hardware([0.0], [-0.0], oracle.BOUNDED,
                                      float(np.finfo(np.float32).tiny), 0.0, 1)
    assert rc == 0 and rep["max_abs"] == 0.0 and rep["max_ulp"] == 1
    rc, rep = oracle.compare_hardware([2.0], [rv.bits_f32(0x40000002)], oracle.BOUNDED, 1.0, 1.0, 1)
    assert rc == oracle.ERR_MISMATCH and rep["max_ulp"] == 2
    rc, _ = oracle.compare_hardware([2.0], [float("nan")], oracle.BOUNDED, 1.0, 1.0, 1)
    assert rc == oracle.ERR_NONFINITE


def test_nine_vector_corpus_digest_is_pinned(oracle):
    """numerical_contract.rs:488-519: FNV-1a over names, dims, strides (usize
    LE), A/B bits, C bits, alpha/beta bits and the expected output bits."""
    h = 0xCBF29CE484222325
    for name, spec, a, b, c, alpha, beta, policy in rv.gemm_corpus_v1():
        m, n, k, lda, ldb, ldc = spec
        h = rv.fnv1a(h, name.encode())
        for val in (m, n, k, lda, ldb, ldc):
            h = rv.fnv1a(h, int(val).to_bytes(8, "little"))
        for bits in list(a) + list(b):
            h = rv.fnv1a(h, int(bits).to_bytes(2, "little"))
        for bits in f32bits(np.array(c, np.float32)):
            h = rv.fnv1a(h, bits.to_bytes(4, "little"))
        h = rv.fnv1a(h, rv.f32_bits(alpha).to_bytes(4, "little"))
        h = rv.fnv1a(h, rv.f32_bits(beta).to_bytes(4, "little"))
        rc, out = oracle.build_hardware_expectation(m, n, k, lda, ldb, ldc, a, b, c, alpha, beta)
        assert rc == 0, name
        for bits in f32bits(out):
            h = rv.fnv1a(h, bits.to_bytes(4, "little"))
        # every case self-compares under its own policy
        if policy is None:
            assert oracle.compare_hardware(out, out, oracle.EXACT_BITS)[0] == 0
        else:
            assert oracle.compare_hardware(out, out, oracle.BOUNDED, *policy)[0] == 0
    assert h == rv.CORPUS_DIGEST


# ---- general tiled schedule (general_reference.rs) -----------------------------

def test_xor4_is_a_row_permutation(oracle):
    for r in range(16):
        phys = sorted(oracle.row_major_xor4(r, c)[1] for c in range(16))
        assert phys == list(range(r * 16, r * 16 + 16))
    assert oracle.row_major_xor4(16, 0)[0] == oracle.ERR_SHAPE


def _bf16_value(i):
    return [0x3F00, 0x3F80, 0xBF80, 0x4000][i % 4]


def test_tiled_reference_matches_scalar_contract(oracle):
    """general_plan.rs:294-360"""
    for m in range(6):
        for n in range(6):
            for k in (0, 1, 15, 16, 17, 18):
                lda = k + (k != 0)
                ldb = n + (k != 0 and n != 0)
                ldc = n + (m != 0 and n != 0)
                empty = m == 0 or n == 0
                _, (la, lb, lc) = oracle.gemm_spec_checked(m, n, k, lda, ldb, ldc)
                if empty:
                    la = lb = lc = 0
                a = np.array([_bf16_value(i) for i in range(la)], np.uint16)
                b = np.array([_bf16_value(i + 1) for i in range(lb)], np.uint16)
                c = np.array([float(int(np.fmod(i, 7)) - 3) for i in range(lc)], np.float32)
                rc, tiled, trace = oracle.general_reference_v1(m, n, k, lda, ldb, ldc, a, b, c,
                                                               0.5, -1.0)
                assert rc == 0
                if empty:
                    assert trace["workgroups"] == 0
                    continue
                rc2, scalar = oracle.evaluate_source(m, n, k, lda, ldb, ldc, a, b, c, 0.5, -1.0)
                assert rc2 == 0 and f32bits(tiled) == f32bits(scalar), (m, n, k)
                wg = ((m + 15) // 16) * ((n + 15) // 16)
                assert trace["workgroups"] == wg
                assert trace["output_stores"] == m * n
                assert trace["reduction_phases"] == wg * ((k + 15) // 16)
                assert trace["publish_barriers"] == trace["reduction_phases"]


def test_general_hardware_cases_are_exact_and_traced(oracle):
    for name, dims, strides, alpha, beta in rv.GENERAL_CASES:
        a, b, c = rv.general_case_inputs(dims, strides)
        rc, out, trace = oracle.general_reference_v1(*dims, *strides, a, b, c, alpha, beta)
        assert rc == 0, name
        rc2, scalar = oracle.evaluate_source(*dims, *strides, a, b, c, alpha, beta)
        assert rc2 == 0 and f32bits(out) == f32bits(scalar), name
        # small integer patterns: every sum is exact, so the expectation is
        # the exact rational alpha*AB + beta*C
        m, n, k = dims
        lda, ldb, ldc = strides
        af = oracle.bf16_to_f32(a)
        bf = oracle.bf16_to_f32(b)
        for i in range(m):
            for j in range(n):
                s = sum(Fraction(float(af[i * lda + d])) * Fraction(float(bf[d * ldb + j]))
                        for d in range(k))
                exact = Fraction(alpha) * s + Fraction(beta) * Fraction(float(c[i * ldc + j]))
                assert Fraction(float(out[i * n + j])) == exact
    a, b, c = rv.general_case_inputs((17, 19, 18), (23, 29, 31))
    rc, _, trace = oracle.general_reference_v1(17, 19, 18, 23, 29, 31, a, b, c, 1.0, 0.0)
    assert trace["a_zero_fills"] > 0 and trace["b_zero_fills"] > 0
    assert trace["c_predicated_stores"] > 0
    assert oracle.general_reference_v1(17, 19, 18, 23, 29, 31, a[:-1], b, c, 1.0, 0.0)[0] == \
        oracle.ERR_LENGTH


# ---- scalar GEMM (scalar_gemm_v1/src/harness.rs) -------------------------------

def test_scalar_gemm_kats(oracle):
    kat = rv.SCALAR_KAT
    assert oracle.scalar_gemm(2, 3, 2, kat["a"], kat["b"]).tolist() == kat["out"]
    assert all(b == 0 for b in f32bits(oracle.scalar_gemm(2, 3, 0, [], [])))
    fd = rv.FMA_DISTINGUISHING
    seq = oracle.scalar_gemm(1, 1, 2, fd["a"], fd["b"])
    assert f32bits(seq) == [0]
    contracted = Fraction(-1) + Fraction(1 + rv.EPS) * Fraction(1 - rv.EPS)
    assert contracted == -Fraction(2) ** -46  # an FMA would return -2^-46, not +0


def test_scalar_inputs_closed_form(oracle):
    a, b = oracle.scalar_gemm_inputs(21, 35)
    assert a.tolist() == [((i * 17) % 29 - 14.0) * 0.125 for i in range(21)]
    assert b.tolist() == [((i * 11) % 31 - 15.0) * 0.0625 for i in range(35)]


# ---- large-shape evaluation forms are bit-identical to the restatement --------

def test_nt_rows_and_points_match_arithmetic_oracle(oracle):
    rng = np.random.default_rng(5)
    for m, n, k in ((5, 7, 3), (16, 33, 64), (9, 16, 130)):
        a = oracle.bf16_from_f32(rng.standard_normal(m * k).astype(np.float32))
        b_kn = oracle.bf16_from_f32(rng.standard_normal(k * n).astype(np.float32))
        rc, ref = oracle.tiled_gemm_arithmetic_v1(m, n, k, a, b_kn)
        b_nk = np.ascontiguousarray(b_kn.reshape(k, n).T).ravel()
        rows = oracle.gemm_bf16_nt_rows(m, n, k, a, b_nk, 0, m, threads=3)
        assert f32bits(rows) == f32bits(ref)
        part = oracle.gemm_bf16_nt_rows(m, n, k, a, b_nk, 2, m - 1, threads=2)
        assert f32bits(part) == f32bits(ref[2 * n:(m - 1) * n])
        ii = rng.integers(0, m, 11)
        jj = rng.integers(0, n, 11)
        pts = oracle.gemm_bf16_nt_points(k, a.reshape(m, k)[ii], b_nk.reshape(n, k)[jj])
        assert f32bits(pts) == f32bits(ref.reshape(m, n)[ii, jj])


def test_f32_rows_match_scalar_gemm(oracle):
    rng = np.random.default_rng(6)
    for m, n, k in ((3, 5, 7), (17, 40, 33)):
        a = rng.uniform(-1, 1, m * k).astype(np.float32)
        b = rng.uniform(-1, 1, k * n).astype(np.float32)
        ref = oracle.scalar_gemm(m, n, k, a, b)
        assert f32bits(oracle.gemm_f32_rows(m, n, k, a, b, 0, m, threads=4)) == f32bits(ref)


# ---- counter-based generators ------------------------------------------------

def test_counter_generators_closed_form(oracle):
    n = 200000
    x = oracle.fill_normal_f32(n, 7, 11, 1.0)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.var()) - 1.0) < 0.01
    assert float(np.abs(x).max()) <= 6.0
    # every value is an integer multiple of 2^-16 (exact construction)
    assert np.all(np.fmod(x * 65536.0, 1.0) == 0)
    u = oracle.fill_uniform_f32(n, 3, 5)
    assert float(u.min()) >= -1.0 and float(u.max()) < 1.0
    assert abs(float(u.mean())) < 0.01
    # first_index offsets address the same counter stream
    assert np.array_equal(oracle.fill_normal_f32(10, 7, 11, 1.0, first=5), x[5:15])
    xb = oracle.fill_normal_bf16(1000, 7, 11, 0.5)
    assert np.array_equal(xb, oracle.bf16_from_f32(x[:1000] * np.float32(0.5)))
    # the hash is the reference's mix64 (inputs.rs:57-62): SplitMix64 of 0
    assert oracle.mix64(0) == 0xE220A8397B1DCDAF
