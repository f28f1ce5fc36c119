"""GPU parity tests for the GEMM family, through the C-ABI, against the CPU
oracle restatements (oracle/).

Bars: bit-exact where the reference's hardware tests
are bit-exact (dyadic/integer inputs, the sequential scalar recurrence);
otherwise the reference's bounded policies, and max|y - yhat| / max|yhat|
<= 1e-2 for bf16 outputs, <= 1e-5 for fp32 outputs.
"""
from __future__ import annotations

import numpy as np
import pytest

from golden import reference_vectors as rv
from gpu_util import GUARD, Guarded, assert_same, bf16_to_f32, rel_err

pytestmark = pytest.mark.gpu

FLT_EPS = np.float32(2.0 ** -23)
FLT_MIN = np.float32(1.17549435e-38)


def _kernels():
    from fe2o3_amd import kernels
    return kernels


# ---- tiled_gemm_lds_slice1 -----------------------------------------------------------

@pytest.mark.parametrize("case", [c[0] for c in rv.lds_tile_cases()])
def test_slice1_six_cases(gpu, oracle, case):
    """crates/fe2o3-hsa-runtime/tests/tiled_gemm_lds_v1_hardware.rs:778-979:
    exact cases bit-exact, the others within 64*eps*sum|p| + FLT_MIN of the
    f64 sum; guards intact, inputs unchanged."""
    name, a, b, exact = next(c for c in rv.lds_tile_cases() if c[0] == case)
    a = np.array(a, np.uint16)
    b = np.array(b, np.uint16)
    ga, gb = Guarded(gpu, a), Guarded(gpu, b)
    gc = Guarded(gpu, np.full(256, np.nan, np.float32))
    k = _kernels().tiled_gemm_lds_slice1_gpu.Kernel.load(gpu)
    k.prepare(ga.body, gb.body, gc.body).launch()
    got = gc.download()
    assert ga.unchanged() and gb.unchanged() and gc.guards_intact()
    af = oracle.bf16_to_f32(a).astype(np.float64).reshape(16, 16)
    bf = oracle.bf16_to_f32(b).astype(np.float64).reshape(16, 16)
    if exact:
        rc, ref = oracle.tiled_gemm_arithmetic_v1(16, 16, 16, a, b)
        assert rc == 0
        assert got.view(np.uint32).tolist() == ref.view(np.uint32).tolist()
    else:
        ref = af @ bf
        bound = 64 * float(FLT_EPS) * (np.abs(af) @ np.abs(bf)) + float(FLT_MIN)
        assert np.all(np.isfinite(got))
        assert np.all(np.abs(got.reshape(16, 16) - ref) <= bound)


def test_slice1_rejects_wrong_lengths_without_writing(gpu):
    from fe2o3_amd.runtime import Fe2o3Error
    a = gpu.to_device(np.zeros(255, np.uint16))
    b = gpu.to_device(np.zeros(256, np.uint16))
    c = Guarded(gpu, np.full(256, 7.0, np.float32))
    with pytest.raises(Fe2o3Error) as e:
        _kernels().tiled_gemm_lds_slice1_gpu.Kernel.load(gpu).prepare(a, b, c.body).launch()
    assert e.value.status == -2
    assert c.unchanged()


def test_moe_expert_tile_matches_slice1_semantics(gpu, oracle):
    """The 16x16x16 expert tile (examples/moe_expert_v1/src/kernel.rs:30-91)
    on the reference's patterned data is exact: compare bits with the
    sequential oracle."""
    acts = rv.moe_expert_activations(oracle.bf16_from_f32)  # 8 tokens x 16 hidden
    a = np.concatenate([np.asarray(acts, np.uint16), np.zeros(128, np.uint16)])  # zero-padded tile
    w = np.asarray(rv.moe_expert_weights(oracle.bf16_from_f32)[:256], np.uint16)  # expert 0
    da, dw = gpu.to_device(a), gpu.to_device(w)
    out = gpu.alloc(256, np.float32)
    _kernels().moe_expert_gemm_bf16_m16_n16_k16_v1_gpu.Kernel.load(gpu).prepare(da, dw, out).launch()
    rc, ref = oracle.tiled_gemm_arithmetic_v1(16, 16, 16, a, w)
    assert rc == 0
    assert out.download().view(np.uint32).tolist() == ref.view(np.uint32).tolist()


# ---- tiled_gemm_general_v1 -------------------------------------------------------------

GENERAL_SCHEDULES = {"reference": "tiled_gemm_general_v1_gpu",
                     "vector-a": "tiled_gemm_general_vector_a_v1_gpu"}


@pytest.mark.parametrize("schedule", list(GENERAL_SCHEDULES))
@pytest.mark.parametrize("case", [c[0] for c in rv.GENERAL_CASES])
def test_general_hardware_matrix_bit_exact(gpu, oracle, case, schedule):
    """examples/tiled_gemm_general_v1/hardware-harness/src/lib.rs:139-253,
    341-396, 1654-1700: the seven profiles under each of the two schedules
    (the reference's 14-case matrix): poisoned bodies, patterned logical
    entries, output bit-exact against the tiled CPU schedule, every
    non-logical C element (stride padding) untouched, inputs unchanged,
    guards intact."""
    name, dims, strides, alpha, beta = next(c for c in rv.GENERAL_CASES if c[0] == case)
    m, n, k = dims
    lda, ldb, ldc = strides
    a, b, c = rv.general_case_inputs(dims, strides)
    rc, out, _ = oracle.general_reference_v1(m, n, k, lda, ldb, ldc, a, b, c, alpha, beta)
    assert rc == 0
    expected = c.copy()
    for r in range(m):
        expected[r * ldc:r * ldc + n] = out[r * n:(r + 1) * n]
    ga, gb, gc = Guarded(gpu, a), Guarded(gpu, b), Guarded(gpu, c)
    getattr(_kernels(), GENERAL_SCHEDULES[schedule]).Kernel.load(gpu).prepare(
        ga.body, gb.body, gc.body, m, n, k, lda, ldb, ldc, alpha, beta).launch()
    got = gc.download()
    assert_same(got, expected, case)
    assert ga.unchanged() and gb.unchanged() and gc.guards_intact()


@pytest.mark.parametrize("dims,strides,alpha,beta", [
    ((1, 1, 1), (1, 1, 1), 1.0, 0.0),
    ((65, 63, 97), (101, 64, 70), 0.75, -0.5),
    ((128, 256, 320), (320, 256, 256), 1.0, 1.0),
    ((200, 130, 77), (77, 131, 140), -2.0, 0.125),
])
def test_general_random_within_tolerance(gpu, oracle, dims, strides, alpha, beta):
    """Random bf16 inputs: MFMA summation order differs from the sequential
    recurrence; rel-err <= 1e-5 (fp32 outputs).  The vectorized-A schedule
    gives the same bits as the reference schedule (aligned and misaligned
    A rows, tails)."""
    m, n, k = dims
    lda, ldb, ldc = strides
    rng = np.random.default_rng(m * 7919 + n * 31 + k)
    la, lb, lc = (m - 1) * lda + k, (k - 1) * ldb + n, (m - 1) * ldc + n
    a = oracle.bf16_from_f32(rng.standard_normal(la).astype(np.float32))
    b = oracle.bf16_from_f32(rng.standard_normal(lb).astype(np.float32))
    c = rng.standard_normal(lc).astype(np.float32)
    rc, out, _ = oracle.general_reference_v1(m, n, k, lda, ldb, ldc, a, b, c, alpha, beta)
    assert rc == 0
    gc = Guarded(gpu, c)
    _kernels().tiled_gemm_general_v1_gpu.Kernel.load(gpu).prepare(
        gpu.to_device(a), gpu.to_device(b), gc.body, m, n, k, lda, ldb, ldc, alpha, beta).launch()
    got = gc.download()
    rows = np.concatenate([got[r * ldc:r * ldc + n] for r in range(m)])
    assert rel_err(rows, out) <= 1e-5
    assert gc.guards_intact()
    gv = Guarded(gpu, c)
    _kernels().tiled_gemm_general_vector_a_v1_gpu.Kernel.load(gpu).prepare(
        gpu.to_device(a), gpu.to_device(b), gv.body, m, n, k, lda, ldb, ldc, alpha,
        beta).launch()
    assert gv.guards_intact()
    assert_same(gv.download(), got, "vector-a schedule vs reference schedule")
    # stride padding of C untouched
    for r in range(m - 1):
        assert got[r * ldc + n:(r + 1) * ldc].tobytes() == c[r * ldc + n:(r + 1) * ldc].tobytes()


@pytest.mark.parametrize("dims,strides,alpha,beta", [
    ((300, 520, 512), (520, 528, 530), 1.5, 0.5),
    ((256, 256, 64), (64, 256, 256), 1.0, 0.0),
    ((1000, 264, 1024), (1032, 264, 270), -0.75, 2.0),
    ((17, 1000, 128), (136, 1003, 1003), 1.0, 1.0),
    ((64, 300, 64), (64, 304, 301), 0.5, -1.0),  # last column chunk reads B's padding
    ((3000, 2900, 128), (136, 2904, 2910), 1.25, -0.5),  # 144 tiles of 256: the 256x256 tile
    # K not a multiple of 64: the partial last stage (A's chunks and B's rows
    # past K masked to zeros)
    ((300, 520, 520), (528, 528, 530), 1.5, 0.5),
    ((256, 384, 72), (72, 384, 390), -1.0, 0.25),
    ((3000, 2900, 200), (200, 2904, 2910), 0.75, 1.0),
    # K not a multiple of 8: A repacked even when aligned
    ((300, 520, 77), (80, 520, 530), 1.0, -0.5),
    # B's stride not a multiple of 8: B repacked
    ((300, 260, 256), (264, 261, 270), 2.0, 0.0),
    # both repacked, K not a multiple of 64 (B's repacked rows end inside the
    # last stage)
    ((200, 130, 77), (77, 131, 140), -2.0, 0.125),
])
def test_general_pipelined_tile_matches_staged_kernel(gpu, oracle, dims, strides, alpha, beta):
    """One GEMM three ways, the same bits: the pipelined tiles on the
    operands as given; the same with A two bytes past a 16-byte boundary
    (the tiles cannot read it in place, so it is repacked into aligned,
    zero-padded rows first when M and N reach 128); and the 64x64 staged
    kernel, reached through row strips of 64 (below the repack size), the
    reference's schedule.  Also with NaN and infinity in A's and B's stride
    padding; C's padding untouched; rel-err <= 1e-5 against the tiled CPU
    schedule."""
    m, n, k = dims
    lda, ldb, ldc = strides
    rng = np.random.default_rng(m + n + k)
    la, lb, lc = (m - 1) * lda + k, (k - 1) * ldb + n, (m - 1) * ldc + n
    a = oracle.bf16_from_f32(rng.standard_normal(la).astype(np.float32))
    b = oracle.bf16_from_f32(rng.standard_normal(lb).astype(np.float32))
    for r in range(m - 1):  # A's padding: NaN and infinity payloads
        a[r * lda + k:(r + 1) * lda] = np.where(np.arange(lda - k) % 2, 0x7F80, 0x7FC1)
    for r in range(k - 1):
        b[r * ldb + n:(r + 1) * ldb] = 0xFF80
    c = rng.standard_normal(lc).astype(np.float32)
    kern = _kernels().tiled_gemm_general_v1_gpu.Kernel.load(gpu)
    gb = gpu.to_device(b)
    gc = Guarded(gpu, c)
    kern.prepare(gpu.to_device(a), gb, gc.body, m, n, k, lda, ldb, ldc, alpha, beta).launch()
    assert gc.guards_intact()
    got = gc.download()
    # the same A two bytes past a 16-byte boundary
    a_off = Guarded(gpu, np.concatenate([np.zeros(1, np.uint16), a]))
    gr = Guarded(gpu, c)
    kern.prepare(a_off.full.view(65, la), gb, gr.body, m, n, k, lda, ldb, ldc, alpha,
                 beta).launch()
    assert gr.guards_intact() and a_off.unchanged()
    assert_same(gr.download(), got, "A at a 2-byte offset vs in place")
    # the staged kernel, 64 rows at a time (strips of C, A and C offset by rows)
    ga_s = gpu.to_device(a)
    gs = gpu.to_device(c)
    for r0 in range(0, m, 64):
        rows = min(64, m - r0)
        kern.prepare(ga_s.view(r0 * lda, (rows - 1) * lda + k), gb,
                     gs.view(r0 * ldc, (rows - 1) * ldc + n), rows, n, k, lda, ldb, ldc, alpha,
                     beta).launch()
    assert_same(gs.download(), got, "pipelined tile vs staged kernel")
    for r in range(m - 1):
        assert got[r * ldc + n:(r + 1) * ldc].tobytes() == c[r * ldc + n:(r + 1) * ldc].tobytes()
    rows = np.concatenate([got[r * ldc:r * ldc + n] for r in range(m)])
    rc, out, _ = oracle.general_reference_v1(m, n, k, lda, ldb, ldc, a, b, c, alpha, beta)
    assert rc == 0
    assert rel_err(rows, out) <= 1e-5


@pytest.mark.parametrize("m,n,k", [(6144, 6144, 128), (6000, 6100, 192)])
def test_general_tail_round_matches_row_blocks(gpu, m, n, k):
    """576 tiles of 256x256 (the last 64 as 128x128 quarters after two full
    rounds), alpha/beta with a nonzero C: the same C computed as row blocks
    of 2048 (no tail) is bit-identical."""
    kern = _kernels()
    lda, ldb, ldc = k + 8, (n + 15) // 8 * 8, n + 4  # A and B rows 16-byte aligned
    da = gpu.alloc((m - 1) * lda + k, np.uint16)
    db = gpu.alloc((k - 1) * ldb + n, np.uint16)
    kern.fill_normal_bf16(da, 14, 0xA, 1.0)
    kern.fill_normal_bf16(db, 14, 0xB, 1.0)
    c0 = np.random.default_rng(m).standard_normal((m - 1) * ldc + n).astype(np.float32)
    K = kern.tiled_gemm_general_v1_gpu.Kernel.load(gpu)
    gc = Guarded(gpu, c0)
    K.prepare(da, db, gc.body, m, n, k, lda, ldb, ldc, 1.25, 0.5).launch()
    assert gc.guards_intact()
    whole = gc.download()
    for r0 in range(0, m, 2048):
        rows = min(2048, m - r0)
        span = (rows - 1) * ldc + n
        part = gpu.to_device(c0[r0 * ldc:r0 * ldc + span])
        K.prepare(da.view(r0 * lda, (rows - 1) * lda + k), db, part, rows, n, k, lda, ldb, ldc,
                  1.25, 0.5).launch()
        got = part.download()
        for r in range(rows):
            assert got[r * ldc:r * ldc + n].tobytes() == \
                whole[(r0 + r) * ldc:(r0 + r) * ldc + n].tobytes(), (r0, r)


def test_general_rejects_small_stride_and_short_slice(gpu):
    from fe2o3_amd.runtime import Fe2o3Error
    a = gpu.to_device(np.zeros(64, np.uint16))
    b = gpu.to_device(np.zeros(64, np.uint16))
    c = Guarded(gpu, np.full(64, 3.0, np.float32))
    K = _kernels().tiled_gemm_general_v1_gpu.Kernel.load(gpu)
    with pytest.raises(Fe2o3Error) as e:
        K.prepare(a, b, c.body, 4, 4, 4, 3, 4, 4, 1.0, 0.0).launch()
    assert e.value.status == -4
    with pytest.raises(Fe2o3Error) as e:
        K.prepare(a, b, c.body, 8, 8, 8, 8, 8, 9, 1.0, 0.0).launch()
    assert e.value.status == -2
    assert c.unchanged()


# ---- scalar_gemm_v1 -----------------------------------------------------------------------

@pytest.mark.parametrize("case", [c[0] for c in rv.SCALAR_CASES])
def test_scalar_hardware_cases_bit_exact(gpu, oracle, case):
    """examples/scalar_gemm_v1/src/harness.rs:148-212: nine cases, the
    reference's deterministic inputs (or the FMA-distinguishing pair), bit
    equality with the sequential unfused oracle."""
    name, m, n, k = next(c for c in rv.SCALAR_CASES if c[0] == case)
    if name == "fma-distinguishing":
        a = np.array(rv.FMA_DISTINGUISHING["a"], np.float32)
        b = np.array(rv.FMA_DISTINGUISHING["b"], np.float32)
    else:
        a, b = oracle.scalar_gemm_inputs(m * k, k * n)
    ref = oracle.scalar_gemm(m, n, k, a, b)
    gc = Guarded(gpu, np.full(m * n, np.nan, np.float32))
    ga, gb = Guarded(gpu, a), Guarded(gpu, b)
    _kernels().scalar_gemm_v1_gpu.Kernel.load(gpu).prepare(ga.body, gb.body, gc.body, m, n, k).launch()
    got = gc.download()
    if m * n:
        assert got.view(np.uint32).tolist() == ref.view(np.uint32).tolist()
    assert gc.guards_intact() and ga.unchanged() and gb.unchanged()
    if name == "fma-distinguishing":
        assert got.view(np.uint32)[0] == 0


def test_scalar_gemm_multi_chunk_bit_exact(gpu, oracle):
    """k over several 256-deep LDS chunks (256 + 256 + 88) and m, n that are
    not multiples of the 16 x 16 workgroup tile: bit equality with the
    sequential unfused oracle, guard bands intact."""
    m, n, k = 33, 47, 600
    a, b = oracle.scalar_gemm_inputs(m * k, k * n)
    ref = oracle.scalar_gemm(m, n, k, a, b)
    gc = Guarded(gpu, np.full(m * n, np.nan, np.float32))
    ga, gb = Guarded(gpu, a), Guarded(gpu, b)
    _kernels().scalar_gemm_v1_gpu.Kernel.load(gpu).prepare(ga.body, gb.body, gc.body, m, n, k).launch()
    assert gc.download().view(np.uint32).tolist() == ref.view(np.uint32).tolist()
    assert gc.guards_intact() and ga.unchanged() and gb.unchanged()


def test_scalar_kat(gpu):
    a = gpu.to_device(np.array(rv.SCALAR_KAT["a"], np.float32))
    b = gpu.to_device(np.array(rv.SCALAR_KAT["b"], np.float32))
    c = gpu.alloc(6, np.float32)
    _kernels().scalar_gemm_v1_gpu.Kernel.load(gpu).prepare(a, b, c, 2, 3, 2).launch()
    assert c.download().tolist() == rv.SCALAR_KAT["out"]


def test_config1_f32_gemm_256_bit_exact(gpu, oracle):
    """f32 C = A.B, M=N=K=256, A,B ~ U[-1,1] from seed 0,
    row-major; the scalar recurrence makes it bit-exact (stronger than the
    1e-5 bar)."""
    m = n = k = 256
    a = oracle.fill_uniform_f32(m * k, 0, 0xA)
    b = oracle.fill_uniform_f32(k * n, 0, 0xB)
    da = gpu.alloc(m * k, np.float32)
    db = gpu.alloc(k * n, np.float32)
    kern = _kernels()
    kern.fill_uniform_f32(da, 0, 0xA)
    kern.fill_uniform_f32(db, 0, 0xB)
    assert da.download().tobytes() == a.tobytes()  # device generator reproduces the oracle's
    c = gpu.alloc(m * n, np.float32)
    kern.scalar_gemm_v1_gpu.Kernel.load(gpu).prepare(da, db, c, m, n, k).launch()
    ref = oracle.scalar_gemm(m, n, k, a, b)
    assert_same(c.download(), ref, "config1")


# ---- bf16 NT GEMM ---------------------------------------------------------------------------

def _nt_case(gpu, oracle, m, n, k, seed, rows=None):
    kern = _kernels()
    scale = 1.0 / np.sqrt(k)
    da = gpu.alloc(m * k, np.uint16)
    db = gpu.alloc(n * k, np.uint16)
    kern.fill_normal_bf16(da, seed, 0xA, scale)
    kern.fill_normal_bf16(db, seed, 0xB, scale)
    dc = Guarded(gpu, np.full(m * n, 0x7FDE, np.uint16))
    kern.gemm_bf16_nt_gpu.Kernel.load(gpu).prepare(da, db, dc.body, m, n, k).launch()
    got = bf16_to_f32(dc.download()).reshape(m, n)
    assert dc.guards_intact()
    a = da.download()
    b = db.download()
    if rows is None:
        rows = range(m)
    rows = list(rows)
    ref = np.stack([oracle.gemm_bf16_nt_rows(m, n, k, a, b, r, r + 1) for r in rows]) \
        if len(rows) < m else oracle.gemm_bf16_nt_rows(m, n, k, a, b, 0, m).reshape(m, n)
    sub = got[rows]
    err = rel_err(sub, ref)
    assert err <= 1e-2, err
    # per element: within one bf16 rounding of the fp32 oracle (plus a small
    # absolute allowance for the differing fp32 summation order)
    assert np.all(np.abs(sub - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-3 * np.max(np.abs(ref)))
    return a, b


def test_fill_normal_bf16_matches_oracle(gpu, oracle):
    d = gpu.alloc(100_003, np.uint16)
    _kernels().fill_normal_bf16(d, 7, 0x5EED, 0.125, first=12345)
    assert d.download().tobytes() == oracle.fill_normal_bf16(100_003, 7, 0x5EED, 0.125, 12345).tobytes()


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (17, 33, 65), (64, 64, 32), (100, 300, 200),
                                   (255, 257, 130)])
def test_gemm_bf16_nt_generic_shapes(gpu, oracle, m, n, k):
    _nt_case(gpu, oracle, m, n, k, seed=3)


# K steps of 64: k = 64 is the first step alone (tail only), 128 the first
# two-step group alone, 192 and 320 whole groups plus a one-step tail.  Up to
# 128 tiles of 256x256 the GEMM runs on 128x128 tiles: three-stage up to 256
# of them, two-stage beyond (4096 x 2048: 512 small tiles).
@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (256, 256, 128), (256, 512, 256),
                                   (512, 768, 1024), (1024, 256, 4096), (256, 256, 320),
                                   (512, 256, 192), (4096, 2048, 128)])
def test_gemm_bf16_nt_fast_path(gpu, oracle, m, n, k):
    _nt_case(gpu, oracle, m, n, k, seed=1)


@pytest.mark.parametrize("m,n,k,which", [(512, 384, 1000, "a"), (512, 384, 1000, "b"),
                                         (384, 640, 4096, "ab"), (4096, 4096, 4096, "a")])
def test_gemm_bf16_nt_misaligned_operands_match_aligned(gpu, m, n, k, which):
    """A and/or B two bytes past a 16-byte boundary: their rows are copied
    into aligned scratch and the pipelined tile runs on the copies, so C is
    bit-identical to the aligned operands' (inputs unchanged, C's guards
    intact)."""
    kern = _kernels()
    da, db = gpu.alloc(m * k, np.uint16), gpu.alloc(n * k, np.uint16)
    kern.fill_normal_bf16(da, 9, 0xA, 1.0 / np.sqrt(k))
    kern.fill_normal_bf16(db, 9, 0xB, 1.0 / np.sqrt(k))
    prep = kern.gemm_bf16_nt_gpu.Kernel.load(gpu)
    want = gpu.alloc(m * n, np.uint16)
    prep.prepare(da, db, want, m, n, k).launch()
    ha, hb = da.download(), db.download()
    offs = {}
    for key, host in (("a", ha), ("b", hb)):
        if key in which:
            offs[key] = Guarded(gpu, np.concatenate([np.zeros(1, np.uint16), host]))
    ga = offs["a"].full.view(GUARD + 1, m * k) if "a" in offs else da
    gb = offs["b"].full.view(GUARD + 1, n * k) if "b" in offs else db
    got = Guarded(gpu, np.full(m * n, 0x7FDE, np.uint16))
    prep.prepare(ga, gb, got.body, m, n, k).launch()
    assert got.guards_intact() and all(o.unchanged() for o in offs.values())
    assert_same(got.download(), want.download(), f"{which} at a 2-byte offset vs aligned")


@pytest.mark.parametrize("m,n,k", [(300, 260, 1003), (256, 512, 4097), (1024, 1024, 77),
                                   (128, 128, 9)])
def test_gemm_bf16_nt_odd_k_repacked(gpu, oracle, m, n, k):
    """K not a multiple of 8 (rows not 16-byte aligned): both operands are
    repacked into rows of K rounded up to 8 and the tile runs on them."""
    _nt_case(gpu, oracle, m, n, k, seed=4)


# M or N not a multiple of 256 with whole 64-k stages: edge tiles of the
# pipelined kernel (clamped operand rows, element-wise masked stores)
@pytest.mark.parametrize("m,n,k", [(300, 520, 512), (257, 255, 128), (1, 1000, 64),
                                   (1000, 264, 1024), (4000, 4000, 256), (4000, 2000, 128)])
def test_gemm_bf16_nt_edge_tiles(gpu, oracle, m, n, k):
    rows = None if m * n <= 1_100_000 else [0, 255, 256, 1999, 3839, 3840, 3999]
    _nt_case(gpu, oracle, m, n, k, seed=6, rows=rows)


# K a multiple of 8 but not of 64: the pipelined tiles' partial last stage
# (chunks past K load zeros) on every launch form: 128x128 small grids
# (three- and two-stage), 256x256 tiles, tail quarters
@pytest.mark.parametrize("m,n,k", [(256, 256, 8), (512, 768, 72), (1000, 264, 1000),
                                   (4096, 2048, 136), (4096, 4096, 4000), (6144, 6144, 200)])
def test_gemm_bf16_nt_k_tail(gpu, oracle, m, n, k):
    rows = None if m * n <= 1_100_000 else [0, 255, 256, 1999, 2048, m - 1]
    _nt_case(gpu, oracle, m, n, k, seed=8, rows=rows)


def test_gemm_bf16_nt_k_tail_matches_zero_padded_k(gpu):
    """K = 4000 against the same operands zero-padded to K = 4032 (whole
    stages, the plain tile): the partial stage's zero chunks are exactly the
    padding, so C is bit-identical."""
    kern = _kernels()
    m = n = 1024
    k, kp = 4000, 4032
    da, db = gpu.alloc(m * k, np.uint16), gpu.alloc(n * k, np.uint16)
    kern.fill_normal_bf16(da, 9, 0xA, 1.0 / 64)
    kern.fill_normal_bf16(db, 9, 0xB, 1.0 / 64)
    a = da.download().reshape(m, k)
    b = db.download().reshape(n, k)
    ap = np.zeros((m, kp), np.uint16)
    bp = np.zeros((n, kp), np.uint16)
    ap[:, :k], bp[:, :k] = a, b
    dc, dcp = gpu.alloc(m * n, np.uint16), gpu.alloc(m * n, np.uint16)
    kern.gemm_bf16_nt_gpu.Kernel.load(gpu).prepare(da, db, dc, m, n, k).launch()
    kern.gemm_bf16_nt_gpu.Kernel.load(gpu).prepare(gpu.to_device(ap.ravel()),
                                                   gpu.to_device(bp.ravel()), dcp, m, n,
                                                   kp).launch()
    assert_same(dc.download(), dcp.download(), "K 4000 vs zero-padded K 4032")


def test_gemm_bf16_nt_small_grid_matches_large_tiles(gpu):
    """The same 2048 rows of A against the same B: at M = 2048 (64 tiles of
    256x256, so 128x128 tiles run) and inside M = 4352 (136 tiles, the
    256x256 tile), on whole and on edge shapes.  Every output gets the same
    MFMAs in the same k order on both tiles: the rows are bit-identical."""
    kern = _kernels()
    for n, k in ((2048, 512), (2000, 320)):
        big = 4352
        da = gpu.alloc(big * k, np.uint16)
        db = gpu.alloc(n * k, np.uint16)
        kern.fill_normal_bf16(da, 12, 0xA, 1.0 / np.sqrt(k))
        kern.fill_normal_bf16(db, 12, 0xB, 1.0 / np.sqrt(k))
        K = kern.gemm_bf16_nt_gpu.Kernel.load(gpu)
        c_big = gpu.alloc(big * n, np.uint16)
        K.prepare(da, db, c_big, big, n, k).launch()
        c_small = gpu.alloc(2048 * n, np.uint16)
        K.prepare(da.view(0, 2048 * k), db, c_small, 2048, n, k).launch()
        assert_same(c_small.download(), c_big.download()[:2048 * n], f"n={n} k={k}")


# 6144 x 6144 x 8192: operands of 192 MiB, so the full rounds store C through
# LDS (the staged epilogue) while the tail quarters store it directly
@pytest.mark.parametrize("m,n,k", [(6144, 6144, 256), (6000, 6100, 192), (4096, 14336, 128),
                                   (6144, 6144, 8192)])
def test_gemm_bf16_nt_tail_round_matches_row_blocks(gpu, m, n, k):
    """576 (or 896) tiles of 256x256: the full rounds on the 256x256 tile and
    the last 64 (128) tiles as 128x128 quarters.  The same C computed as row
    blocks of 2048 (at most 200 tiles each, no tail) is bit-identical; the
    guards around C are untouched."""
    kern = _kernels()
    da = gpu.alloc(m * k, np.uint16)
    db = gpu.alloc(n * k, np.uint16)
    kern.fill_normal_bf16(da, 13, 0xA, 1.0 / np.sqrt(k))
    kern.fill_normal_bf16(db, 13, 0xB, 1.0 / np.sqrt(k))
    K = kern.gemm_bf16_nt_gpu.Kernel.load(gpu)
    c = Guarded(gpu, np.full(m * n, 0x7FDE, np.uint16))
    K.prepare(da, db, c.body, m, n, k).launch()
    assert c.guards_intact()
    whole = c.download()
    for r0 in range(0, m, 2048):
        rows = min(2048, m - r0)
        part = gpu.alloc(rows * n, np.uint16)
        K.prepare(da.view(r0 * k, rows * k), db, part, rows, n, k).launch()
        assert_same(part.download(), whole[r0 * n:(r0 + rows) * n], f"rows {r0}..{r0 + rows}")


def test_gemm_bf16_nt_whole_tiles_unaligned_c(gpu, oracle):
    """Whole tiles but C at an odd element offset: the edge form, 2-byte
    stores; every output against the oracle and the neighbours untouched."""
    m, n, k = 256, 512, 192
    kern = _kernels()
    da, db = gpu.alloc(m * k, np.uint16), gpu.alloc(n * k, np.uint16)
    kern.fill_normal_bf16(da, 8, 0xA, 1.0 / np.sqrt(k))
    kern.fill_normal_bf16(db, 8, 0xB, 1.0 / np.sqrt(k))
    c = Guarded(gpu, np.full(m * n + 1, 0x7FDE, np.uint16))
    body = c.full.view(65, m * n)  # one element past the guard: 2-byte aligned only
    kern.gemm_bf16_nt_gpu.Kernel.load(gpu).prepare(da, db, body, m, n, k).launch()
    full = c.full.download()
    assert c.guards_intact() and full[64] == 0x7FDE
    got = bf16_to_f32(full[65:65 + m * n]).reshape(m, n)
    ref = oracle.gemm_bf16_nt_rows(m, n, k, da.download(), db.download(), 0, m).reshape(m, n)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-3 * np.max(np.abs(ref)))


def test_gemm_bf16_nt_more_tiles_than_cus(gpu, oracle):
    """264 output tiles (more than one per CU): sampled rows of every tile
    row against the oracle."""
    m, n, k = 2048, 8448, 640
    rows = [t * 256 + (t * 53) % 256 for t in range(8)] + [0, 2047]
    _nt_case(gpu, oracle, m, n, k, seed=4, rows=rows)


def test_gemm_bf16_nt_staged_epilogue(gpu, oracle):
    """Operands of 243 MB, above the size at which C leaves through LDS with
    nontemporal stores: whole rows of every tile row against the oracle."""
    m, n, k = 1024, 28672, 4096
    rows = [t * 256 + (t * 97) % 256 for t in range(4)] + [0, 511, 1023]
    _nt_case(gpu, oracle, m, n, k, seed=5, rows=rows)


def test_gemm_bf16_nt_config2_4096(gpu, oracle):
    """BASELINE config 2 (bf16 4096^3, A row-major, B column-major,
    N(0,1)/sqrt(K), seed 1): every one of the 16.8M outputs against the
    sequential fp32 oracle (rel-err and per-element bounds)."""
    m = n = k = 4096
    _nt_case(gpu, oracle, m, n, k, seed=1)


@pytest.mark.parametrize("m,n", [(256, 512), (3, 7)])
def test_gemm_bf16_nt_k0_writes_positive_zero(gpu, m, n):
    """K = 0: every output is +0 (the empty sum), the guards untouched."""
    a = gpu.alloc(0, np.uint16)
    b = gpu.alloc(0, np.uint16)
    c = Guarded(gpu, np.full(m * n, 0xFFFF, np.uint16))
    _kernels().gemm_bf16_nt_gpu.Kernel.load(gpu).prepare(a, b, c.body, m, n, 0).launch()
    assert c.guards_intact()
    assert c.download().tolist() == [0] * (m * n)


def test_gemm_bf16_nt_rejects_bad_lengths(gpu):
    from fe2o3_amd.runtime import Fe2o3Error
    a = gpu.alloc(256 * 64, np.uint16)
    b = gpu.alloc(256 * 64, np.uint16)
    c = Guarded(gpu, np.zeros(256 * 255, np.uint16))
    with pytest.raises(Fe2o3Error) as e:
        _kernels().gemm_bf16_nt_gpu.Kernel.load(gpu).prepare(a, b, c.body, 256, 256, 64).launch()
    assert e.value.status == -2
    assert c.unchanged()
