"""Golden data held by the reference's own tests for the dense-compute path.

Every constant below is copied as DATA (inputs and pinned expected outputs)
from the reference test or vector file cited next to it; the constructors
rebuild the reference's deterministic input vectors from the rules those
files state.  Nothing here computes an expected output: the pins are the
reference's numbers, and the oracle under test must reproduce them.
"""
from __future__ import annotations

import struct

import numpy as np

MASK64 = (1 << 64) - 1


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def bits_f32(b: int) -> float:
    return struct.unpack("<f", struct.pack("<I", b))[0]


# ---- examples/tiled_gemm_v1/tests/inputs_oracle.rs:29-59 ----------------------
GENERATOR_PIN = {
    "shape": (2, 3, 2),
    "seed": 0x1234,
    "a_bits": [0x0000, 0x4080, 0xBD80, 0x4040],
    "b_bits": [0xBE80, 0x4040, 0x4040, 0x3E80, 0x4080, 0x3E00],
    "out_bits": [0x3F800000, 0x41800000, 0x3F000000, 0x3F440000, 0x413D0000, 0x3E400000],
}

# inputs.rs:12-29 alphabet (BF16_INPUT_PATTERN_V1)
BF16_INPUT_PATTERN_V1 = [0x0000, 0x3D80, 0xBD80, 0x3E00, 0xBE00, 0x3E80, 0xBE80, 0x3F00,
                         0xBF00, 0x3F80, 0xBF80, 0x4000, 0xC000, 0x4040, 0xC040, 0x4080]

# inputs_oracle.rs:86-159: hostile BF16 classes for evidence admission
HOSTILE_BF16 = [(0x7FC1, "nan"), (0xFFC1, "nan"), (0x7F80, "inf"), (0xFF80, "inf"),
                (0x0001, "subnormal"), (0x807F, "subnormal"), (0x8000, "alphabet"),
                (0x3F40, "alphabet")]

# ---- examples/tiled_gemm_v1/tests/numerical_contract.rs:124-147 -----------------
SOURCE_KAT = {
    "dims": (2, 2, 3), "strides": (3, 2, 3),
    "a": [0x3F80, 0x4000, 0x4040, 0x4080, 0x40A0, 0x40C0],
    "b": [0x40A0, 0x40C0, 0x40E0, 0x4100, 0x4110, 0x4120],
    "c": [4.0, -8.0, float("nan"), 12.0, -16.0],
    "alpha": 0.5, "beta": 0.25,
    "out_bits": [0x41C00000, 0x41C00000, 0x42660000, 0x42680000],
}

# numerical_contract.rs:21-49
ZERO_K_KAT = {
    "dims": (2, 3, 0), "strides": (0, 3, 5),
    "c": [2.0, 4.0, 6.0, float("nan"), float("nan"), 8.0, 10.0, 12.0],
    "alpha": 7.0, "beta": 0.5, "out": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0],
    "padded_spec": ((3, 2, 4, 7, 5, 4), (18, 17, 10)),
}

# numerical_contract.rs:488-519: FNV-1a digest of the nine-vector corpus
CORPUS_DIGEST = 0x6131FB795A3C1C51


def _splitmix64(state):
    state[0] = (state[0] + 0x9E3779B97F4A7C15) & MASK64
    v = state[0]
    v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & MASK64
    return v ^ (v >> 31)


def _packed(m, n, k):
    return (m, n, k, k, n, n)


def gemm_corpus_v1():
    """examples/tiled_gemm_v1/src/numerical_vectors.rs:134-328, in order.
    Each entry: name, spec (m,n,k,lda,ldb,ldc), a, b, c, alpha, beta, policy
    (None = ExactBits, else (max_abs, max_rel, max_ulps))."""
    v = []
    v.append(("zero-signed", _packed(2, 3, 4),
              [0x0000, 0x8000, 0x0000, 0x8000, 0x8000, 0x0000, 0x8000, 0x0000],
              [0x0000, 0x8000, 0x0000, 0x8000, 0x0000, 0x8000, 0x0000, 0x8000, 0x0000, 0x8000,
               0x0000, 0x8000],
              [0.0, -0.0, 0.0, -0.0, 0.0, -0.0], 1.0, 1.0, None))
    v.append(("identity-3x3", _packed(3, 3, 3),
              [0x3F80, 0, 0, 0, 0x3F80, 0, 0, 0, 0x3F80],
              [0x3F00, 0xBF80, 0x4000, 0x4040, 0xC000, 0x3E80, 0x4080, 0x3F80, 0xC040],
              [0.0] * 9, 1.0, 0.0, None))
    v.append(("dyadic-2x2x3", _packed(2, 2, 3),
              [0x3F00, 0xBF80, 0x4000, 0x3E80, 0x4040, 0xC000],
              [0x3F80, 0x3E00, 0xBF00, 0x4000, 0x4080, 0x3F00],
              [0.0] * 4, 1.0, 0.0, None))
    v.append(("cancellation-pairs", _packed(1, 2, 4),
              [0x3F80, 0x3F80, 0x4000, 0x4000],
              [0x4080, 0x4040, 0xC080, 0xC040, 0x3F00, 0xBF00, 0xBF00, 0x3F00],
              [0.0] * 2, 1.0, 0.0, None))
    alphabet = [0xBD80, 0xBE00, 0xBE80, 0xBF00, 0xBF80, 0x0000, 0x3D80, 0x3E00, 0x3E80,
                0x3F00, 0x3F80, 0x4000]
    state = [0x10905EEDD15CA11E]
    a = [alphabet[_splitmix64(state) % 12] for _ in range(5 * 17)]
    b = [alphabet[_splitmix64(state) % 12] for _ in range(17 * 4)]
    v.append(("randomized-seed-109", _packed(5, 4, 17), a, b, [0.0] * 20, 1.0, 0.0,
              (1e-5, 1e-5, 8)))
    # padded-independent-strides: GemmSpec(3,2,4, 7,5,4)
    a_len, b_len, c_len = 2 * 7 + 4, 3 * 5 + 2, 2 * 4 + 2
    a = [0x7FC1] * a_len
    b = [0x7F80] * b_len
    c = [float("nan")] * c_len
    for row in range(3):
        for d in range(4):
            a[row * 7 + d] = [0x3F80, 0x4000, 0xBF80, 0x3F00][(row + d) % 4]
    for d in range(4):
        for col in range(2):
            b[d * 5 + col] = [0x3F00, 0xBF00, 0x4000, 0xC000][d]
    for row in range(3):
        for col in range(2):
            c[row * 4 + col] = 0.0
    v.append(("padded-independent-strides", (3, 2, 4, 7, 5, 4), a, b, c, 1.0, 0.0, None))
    alphabet8 = [0xBE80, 0xBE00, 0x0000, 0x3E00, 0x3E80, 0x3F00, 0xBF00, 0x3F80]
    a = [alphabet8[(i * 5 + i // 7 + 3) % 8] for i in range(17 * 23)]
    b = [alphabet8[(i * 3 + i // 11 + 1) % 8] for i in range(23 * 19)]
    v.append(("tails-m17-n19-k23", _packed(17, 19, 23), a, b, [0.0] * (17 * 19), 1.0, 0.0, None))
    v.append(("alpha-beta-nonzero-c", _packed(2, 3, 3),
              [0x3F80, 0x4000, 0xBF80, 0x3F00, 0xC000, 0x4040],
              [0x3F80, 0x3F00, 0xBF00, 0x4000, 0xC000, 0x3E80, 0x4080, 0x3F80, 0xC080],
              [4.0, -8.0, 12.0, -16.0, 20.0, -24.0], 0.5, 0.25, None))
    v.append(("finite-extremes-and-signed-zero", _packed(6, 1, 1),
              [0x7F7F, 0xFF7F, 0x0080, 0x8080, 0x0000, 0x8000], [0x3F80],
              [0.0, -0.0, 0.0, -0.0, 0.0, -0.0], 1.0, 0.0, None))
    return v


def fnv1a(h: int, data: bytes) -> int:
    for byte in data:
        h ^= byte
        h = (h * 0x100000001B3) & MASK64
    return h


# ---- examples/tiled_gemm_general_v1/hardware-harness/src/lib.rs:139-253 ---------
GENERAL_CASES = [
    ("packed", (16, 16, 16), (16, 16, 16), 1.0, 0.0),
    ("strided-all-tails", (17, 19, 18), (23, 29, 31), 0.5, -1.0),
    ("multi-wg-multi-phase", (33, 35, 33), (37, 41, 43), 2.0, 0.25),
    ("m-tail", (17, 16, 16), (16, 16, 16), -1.0, 1.0),
    ("n-tail", (16, 17, 16), (16, 19, 23), 1.5, -0.5),
    ("k-tail", (16, 16, 17), (21, 19, 16), -0.5, 2.0),
    ("zero-k", (17, 19, 0), (0, 0, 23), 7.0, 0.5),
]
# lib.rs:31-39 poison/guard encodings
A_BODY_POISON, B_BODY_POISON, C_BODY_POISON_BITS = 0x7FC1, 0x7FD1, 0x7FC0C001


def general_pattern(row, col, rf, cf, mod):
    """lib.rs:1640-1648"""
    return float((row * rf + col * cf) % mod) - float(mod // 2)


def general_case_inputs(dims, strides):
    """lib.rs:341-396: poisoned bodies with the logical entries patterned."""
    m, n, k = dims
    lda, ldb, ldc = strides

    def extent(rows, cols, stride):
        return 0 if rows == 0 or cols == 0 else (rows - 1) * stride + cols

    a = np.full(extent(m, k, lda), A_BODY_POISON, np.uint16)
    b = np.full(extent(k, n, ldb), B_BODY_POISON, np.uint16)
    c = np.full(extent(m, n, ldc), C_BODY_POISON_BITS, np.uint32).view(np.float32)
    for r in range(m):
        for d in range(k):
            a[r * lda + d] = f32_bits(general_pattern(r, d, 3, 5, 7)) >> 16
    for d in range(k):
        for col in range(n):
            b[d * ldb + col] = f32_bits(general_pattern(d, col, 2, 3, 5)) >> 16
    for r in range(m):
        for col in range(n):
            c[r * ldc + col] = general_pattern(r, col, 7, 11, 13)
    return a, b, c


# ---- examples/scalar_gemm_v1/src/harness.rs:148-212 ------------------------------
SCALAR_CASES = [("zero-m", 0, 257, 3), ("zero-n", 7, 0, 3), ("zero-k", 3, 5, 0),
                ("one-output", 1, 1, 1), ("wg-minus-one", 1, 255, 3), ("one-wg", 1, 256, 3),
                ("wg-plus-one", 1, 257, 3), ("rectangular", 7, 5, 9),
                ("fma-distinguishing", 1, 1, 2)]
SCALAR_KAT = {"a": [1.0, 2.0, 3.0, 4.0], "b": [5.0, 6.0, 7.0, 8.0, 9.0, 10.0],
              "out": [21.0, 24.0, 27.0, 47.0, 54.0, 61.0]}  # harness.rs:257-266
EPS = 2.0 ** -23
FMA_DISTINGUISHING = {"a": [-1.0, 1.0 + EPS], "b": [1.0, 1.0 - EPS]}  # harness.rs:134-140


# ---- crates/fe2o3-hsa-runtime/tests/tiled_gemm_lds_v1_hardware.rs:778-894 -------
def lds_tile_cases():
    """Six 16x16x16 cases: (name, a[256], b[256], exact)."""
    T = 16
    cases = [("zero", [0] * 256, [0] * 256, True)]
    ia = [0] * 256
    ib = [0] * 256
    pal = [0x3F80, 0xBF80, 0x3F00, 0xBF00, 0x4000, 0xC000]
    for r in range(T):
        ia[r * T + r] = 0x3F80
        for c in range(T):
            ib[r * T + c] = pal[(7 * r + 3 * c) % 6]
    cases.append(("identity", ia, ib, True))
    dp = [0x3F80, 0xBF80, 0x3F00, 0xBF00, 0x3E80, 0xBE80]
    da = [dp[(r + 3 * c) % 6] for r in range(T) for c in range(T)]
    db = [dp[(2 * r + c + 1) % 6] for r in range(T) for c in range(T)]
    cases.append(("dyadic", da, db, True))
    rp = [0x3C80, 0xBC80, 0x3D80, 0xBD80, 0x3E80, 0xBE80, 0x3F00, 0xBF00, 0x3F80, 0xBF80,
          0x4000, 0xC000, 0x4080, 0xC080]
    st = [0x6A09E667F3BCC909]

    def nxt():
        s = st[0]
        s ^= (s << 13) & MASK64
        s ^= s >> 7
        s ^= (s << 17) & MASK64
        st[0] = s
        return rp[s % 14]
    ra = [nxt() for _ in range(256)]
    rb = [nxt() for _ in range(256)]
    cases.append(("deterministic-random", ra, rb, False))
    ca = [0x4100 if (r + d) % 2 == 0 else 0xC100 for r in range(T) for d in range(T)]
    cb = [0x3F80 if (d + c) % 2 == 0 else 0xBF80 for d in range(T) for c in range(T)]
    cases.append(("signed-cancellation", ca, cb, False))
    aa = []
    for r in range(T):
        for d in range(T):
            mag = 0x7F7F if (d & 3) < 2 else 0x0080
            aa.append(mag ^ (0 if (r + d) % 2 == 0 else 0x8000))
    ab = []
    for d in range(T):
        for c in range(T):
            sign = 0 if c % 2 == 0 else 0x8000
            ab.append((0x0080 if (d & 3) in (0, 1) else 0x7F7F) ^ sign)
    cases.append(("adversarial-finite-bf16", aa, ab, False))
    return cases


# ---- examples/flash_attention_v1/src/vectors.rs:18-95 -----------------------------
def flash_vectors_v1():
    E = 128
    out = []
    q, k, v = flash_vectors_v1_f32()
    out.append(("nominal-mixed-sign", q, k, v))
    q = [0.0] * E
    k = [float(i % 19) - 9.0 for i in range(E)]
    v = [(i // 16) * 0.5 + (i % 16) * 0.03125 for i in range(E)]
    out.append(("all-equal-logits", q, k, v))
    q, k, v = [0.0] * E, [0.0] * E, [0.0] * E
    for r in range(8):
        q[r * 16] = 1.0
        k[r * 16] = r * 64.0
        for c in range(16):
            v[r * 16 + c] = r * 10.0 + c
    out.append(("latest-causal-key-dominates", q, k, v))
    q, k, v = [0.0] * E, [0.0] * E, [0.0] * E
    for r in range(8):
        q[r * 16 + r] = 0.5
        k[r * 16 + r] = 0.75
        v[r * 16 + r] = 1.0
    out.append(("causal-mask-weight-probe", q, k, v))
    # The remaining vectors are exact in binary32 whichever precision the
    # expressions are evaluated in.
    res = []
    for name, q, k, v in out:
        res.append((name, _f32_expr(q), _f32_expr(k), _f32_expr(v)))
    return res


def _f32_expr(values):
    return np.array(values, dtype=np.float32)


def flash_vectors_v1_f32():
    """The nominal vector's expressions evaluated step by step in f32, as the
    Rust source does: ((i*17+3)%29) as f32 / 16.0 - 0.75 etc."""
    E = 128
    f = np.float32
    q = np.array([f(f((i * 17 + 3) % 29) / f(16.0)) - f(0.75) for i in range(E)], np.float32)
    k = np.array([f(f((i * 11 + 5) % 31) / f(20.0)) - f(0.70) for i in range(E)], np.float32)
    v = np.array([f(f((i * 7 + 2) % 37) / f(12.0)) - f(1.25) for i in range(E)], np.float32)
    return q, k, v


# ---- examples/row_softmax_v1 ---------------------------------------------------
def softmax_corpus_v1():
    """tests/numerical_contract.rs:66-94 (equal, ramp, dominant, alternating,
    LCG 0x6d2b79f5)."""
    rows = [np.zeros(64, np.float32),
            np.array([i - 32.0 for i in range(64)], np.float32),
            np.array([10001.0 if i == 17 else 10000.0 for i in range(64)], np.float32),
            np.array([8.0 if i % 2 == 0 else -8.0 for i in range(64)], np.float32)]
    state = 0x6D2B79F5
    vals = []
    for _ in range(64):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        vals.append(np.float32(((state >> 8) % 4096)) / np.float32(256.0))
    rows.append(np.array(vals, np.float32))
    return rows


def softmax_production_cases_v1():
    """src/production_release.rs:347-363"""
    normal = np.array([np.float32((i * 17 + 3) % 29) * np.float32(0.25) - np.float32(3.5)
                       for i in range(64)], np.float32)
    equal = np.full(64, 0.5, np.float32)
    dominant = np.full(64, -32.0, np.float32)
    dominant[37] = 32.0
    exceptional = np.zeros(64, np.float32)
    exceptional[11] = np.nan
    return {"normal": normal, "equal": equal, "dominant": dominant, "exceptional": exceptional}


# ---- examples/moe_top2_v1/src/vectors.rs:14-117 ------------------------------------
F32_MAX = float(np.finfo(np.float32).max)
F32_MIN_POS = float(np.finfo(np.float32).tiny)
MOE_VECTORS = {
    "nominal-balanced": [4.0, 3.0, 2.0, 1.0, 1.0, 4.0, 3.0, 2.0, 2.0, 1.0, 4.0, 3.0, 3.0, 2.0,
                         1.0, 4.0] * 2,
    "all-equal-tie-break-and-empty-experts": [1.0] * 32,
    "repeated-logits": [5.0, 5.0, 5.0, 4.0, 1.0, 3.0, 3.0, 3.0, -2.0, -2.0, -2.0, -2.0, 7.0, 6.0,
                        7.0, 6.0, 0.0, -1.0, -1.0, 0.0, 2.0, 2.0, 1.0, 2.0, 8.0, 9.0, 9.0, 8.0,
                        -3.0, -2.0, -3.0, -2.0],
    "stable-capacity-overflow": [10.0, 9.0, 2.0, 1.0, 10.0, 1.0, 9.0, 2.0, 10.0, 2.0, 1.0, 9.0,
                                 10.0, 9.0, 2.0, 1.0, 10.0, 1.0, 9.0, 2.0, 10.0, 2.0, 1.0, 9.0,
                                 10.0, 9.0, 2.0, 1.0, 10.0, 1.0, 9.0, 2.0],
    "empty-experts": [2.0, 1.0, -4.0, -5.0, 2.0, 1.0, -3.0, -6.0, 2.0, 1.0, -2.0, -7.0, 2.0, 1.0,
                      -1.0, -8.0, 2.0, 1.0, -8.0, -1.0, 2.0, 1.0, -7.0, -2.0, 2.0, 1.0, -6.0,
                      -3.0, 2.0, 1.0, -5.0, -4.0],
    "adversarial-finite-values": [F32_MAX, -F32_MAX, F32_MIN_POS, -0.0, -F32_MIN_POS, 0.0,
                                  -F32_MAX, F32_MAX, F32_MAX, F32_MAX, -F32_MAX, -F32_MAX,
                                  -F32_MAX, -0.0, 0.0, F32_MIN_POS, 1.0e30, -1.0e30, 1.0e-30,
                                  -1.0e-30, -42.0, -42.0, -42.0, -43.0, 17.0, 18.0, 17.0, 18.0,
                                  3.5, 3.25, 3.75, 3.0],
}
# tests/oracle.rs:33-89 pinned routing outputs
MOE_PINS = {
    "nominal-balanced": {"requested_counts": [4, 4, 4, 4], "admitted_counts": [4, 4, 4, 4],
                         "expert_offsets": [0, 4, 8, 12, 16]},
    "all-equal-tie-break-and-empty-experts": {
        "top2_pairs": [0, 1], "requested_counts": [8, 8, 0, 0], "admitted_counts": [4, 4, 0, 0],
        "expert_offsets": [0, 4, 8, 8, 8]},
    "stable-capacity-overflow": {"requested0": 8, "expert0_routes": [0, 2, 4, 6],
                                 "dropped_routes": [8, 10, 12, 14]},
    "empty-experts": {"requested_counts": [8, 8, 0, 0]},
}


# ---- examples/moe_expert_v1/tests/pipeline_oracle.rs:15-65 -------------------------
def moe_expert_equal_logits():
    return [1.0] * 32


def moe_expert_balanced_logits():
    lg = [-4.0] * 32
    for t in range(8):
        lg[t * 4 + t % 4] = 4.0
        lg[t * 4 + (t + 1) % 4] = 3.0
    return lg


def moe_expert_activations(bf16_from_f32):
    return bf16_from_f32(np.array([((i % 13) - 6.0) * 0.25 for i in range(128)], np.float32))


def moe_expert_weights(bf16_from_f32):
    vals = []
    for idx in range(4 * 256):
        e, within = idx // 256, idx % 256
        d, o = within // 16, within % 16
        vals.append(1.0 + e * 0.25 if d == o else ((d + o + e) % 5) * 0.03125)
    return bf16_from_f32(np.array(vals, np.float32))


def moe_expert_route_weights():
    return np.array([0.75 if r % 2 == 0 else 0.25 for r in range(16)], np.float32)


# ---- crates/fe2o3-hsa-runtime/tests/flash_attention_v1_hardware.rs:94-117 --------
def flash_hardware_vectors_v1():
    """The hardware test's nominal / equal / dominant vectors (B1 H1 N8 D16)."""
    n, d = 8, 16
    e = n * d
    f = np.float32
    nominal = (np.array([(f(i % 13) - f(6.0)) / f(8.0) for i in range(e)], np.float32),
               np.array([(f(i % 11) - f(5.0)) / f(7.0) for i in range(e)], np.float32),
               np.array([(f(i % 17) - f(8.0)) / f(9.0) for i in range(e)], np.float32))
    equal = (np.zeros(e, np.float32), np.ones(e, np.float32),
             np.array([f(i // d) + f(i % d) / f(32.0) for i in range(e)], np.float32))
    q = np.zeros(e, np.float32)
    k = np.zeros(e, np.float32)
    for r in range(n):
        q[r * d] = 8.0
        k[r * d] = 8.0 if r == 3 else -8.0
    dominant = (q, k, np.array([(f(i % d) - f(7.0)) / f(4.0) for i in range(e)], np.float32))
    return [("nominal", *nominal), ("equal", *equal), ("dominant", *dominant)]


# examples/tiled_gemm_v1/src/contract.rs:458-536 (EDGE_CASES_V1): name, m, n,
# k and the required plan outcome ("no-dispatch", "host-fill", "dispatch", or
# the rejection "m-tail" / "n-tail" / "k-tail")
EDGE_CASES_V1 = [
    ("all-zero", 0, 0, 0, "no-dispatch"),
    ("zero-m-with-k-tail", 0, 17, 3, "no-dispatch"),
    ("zero-n", 32, 0, 16, "no-dispatch"),
    ("zero-k", 16, 32, 0, "host-fill"),
    ("single-tile", 16, 16, 16, "dispatch"),
    ("rectangular-multi-tile", 32, 48, 32, "dispatch"),
    ("three-reduction-tiles", 16, 16, 48, "dispatch"),
    ("m-tail", 17, 16, 16, "m-tail"),
    ("n-tail", 16, 31, 16, "n-tail"),
    ("k-tail-below-one-tile", 16, 16, 15, "k-tail"),
    ("k-tail-after-one-tile", 16, 16, 17, "k-tail"),
]

# examples/tiled_gemm_v1/tests/contract.rs:64-101: empty outputs with extreme
# unused extents plan no dispatch; nonempty extremes overflow the byte
# accounting of A, then B, then C
EXTREME_EMPTY_V1 = [(0, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0, 0xFFFFFFFF),
                    (0, 0, 0xFFFFFFFF), (0, 1, 1), (1, 0, 1), (0, 17, 3), (31, 0, 17)]
BYTE_OVERFLOW_V1 = [(0xFFFFFFFF, 1, 0xFFFFFFFF, "A"), (1, 0xFFFFFFFF, 0xFFFFFFFF, "B"),
                    (0xFFFFFFFF, 0xFFFFFFFF, 1, "C")]
