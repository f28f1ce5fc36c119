"""The reference's GEMM numerical contract judged on GPU outputs.

1. The nine deterministic vectors of
   examples/tiled_gemm_v1/src/numerical_vectors.rs:134-328 run through
   fe2o3_tiled_gemm_general_v1 (strided operands, alpha/beta, padding that
   holds NaN and infinity payloads) and each device output is judged by the
   oracle's build_hardware_expectation + compare_hardware under the vector's
   own policy (ExactBits, or Bounded 1e-5/1e-5/8 ULP for randomized-seed-109),
   numerical_contract.rs:794 and :901-981.  C's padding stays untouched.
2. Every row of EDGE_CASES_V1 (examples/tiled_gemm_v1/src/contract.rs:
   458-536) through fe2o3_tiled_gemm_v1, the multi-tile plan: no dispatch,
   +0 host fill, exact-tile dispatch or the named tail rejection.
3. Exact-tile dispatch shapes (the reference's representative shapes and
   larger ones): bit-exact to the arithmetic oracle on the pinned dyadic
   alphabet of generate_inputs_v1 (every partial sum is exact there, so the
   MFMA order cannot change a bit), and within 1e-5 (the fp32 bar) on
   N(0,1) inputs.
"""
from __future__ import annotations

import numpy as np
import pytest

from golden import reference_vectors as rv
from gpu_util import Guarded, rel_err

pytestmark = pytest.mark.gpu


def _k():
    from fe2o3_amd import kernels
    return kernels


# ---- 1. the nine-vector corpus through the general kernel -----------------------------------

CORPUS = {v[0]: v for v in rv.gemm_corpus_v1()}


@pytest.mark.parametrize("name", list(CORPUS))
def test_corpus_vector_on_general_kernel(gpu, oracle, name):
    _, (m, n, k, lda, ldb, ldc), a, b, c, alpha, beta, policy = CORPUS[name]
    a = np.array(a, np.uint16)
    b = np.array(b, np.uint16)
    c = np.array(c, np.float32)
    rc, expected = oracle.build_hardware_expectation(m, n, k, lda, ldb, ldc, a, b, c, alpha, beta)
    assert rc == 0
    ga, gb, gc = Guarded(gpu, a), Guarded(gpu, b), Guarded(gpu, c)
    _k().tiled_gemm_general_v1_gpu.Kernel.load(gpu).prepare(
        ga.body, gb.body, gc.body, m, n, k, lda, ldb, ldc, alpha, beta).launch()
    assert ga.unchanged() and gb.unchanged() and gc.guards_intact()
    out = gc.download()
    idx = np.array([r * ldc + j for r in range(m) for j in range(n)], np.int64)
    observed = out[idx]
    if policy is None:
        rc, rep = oracle.compare_hardware(expected, observed, oracle.EXACT_BITS)
    else:
        rc, rep = oracle.compare_hardware(expected, observed, oracle.BOUNDED, *policy)
    assert rc == 0, (name, rep)
    # C outside the m x n window (its stride padding) is untouched, bit for bit
    pad = np.ones(c.size, bool)
    pad[idx] = False
    assert out[pad].view(np.uint32).tolist() == c[pad].view(np.uint32).tolist()


# ---- 2. EDGE_CASES_V1 through the multi-tile plan ----------------------------------------------

EDGE = {e[0]: e for e in rv.EDGE_CASES_V1}
CODES = {"m-tail": -24, "n-tail": -25, "k-tail": -26}


@pytest.mark.parametrize("name", list(EDGE))
def test_edge_case_v1(gpu, oracle, name):
    from fe2o3_amd.runtime import Fe2o3Error
    _, m, n, k, outcome = EDGE[name]
    empty = m == 0 or n == 0
    a, b = oracle.generate_inputs_v1(m, n, k, 0x5EED)
    if empty:
        assert a.size == 0 and b.size == 0
    ga, gb = Guarded(gpu, a), Guarded(gpu, b)
    gc = Guarded(gpu, np.full(0 if empty else m * n, np.nan, np.float32))
    prep = _k().tiled_gemm_v1_gpu.Kernel.load(gpu).prepare(ga.body, gb.body, gc.body, m, n, k)
    if outcome in CODES:
        with pytest.raises(Fe2o3Error) as e:
            prep.launch()
        assert e.value.status == CODES[outcome]
        assert gc.unchanged()
        return
    prep.launch()
    assert ga.unchanged() and gb.unchanged() and gc.guards_intact()
    got = gc.download()
    if outcome == "no-dispatch":
        assert got.size == 0
    elif outcome == "host-fill":
        assert got.view(np.uint32).tolist() == [0] * (m * n)  # +0, not -0
    else:
        rc, ref = oracle.tiled_gemm_arithmetic_v1(m, n, k, a, b)
        assert rc == 0
        assert got.view(np.uint32).tolist() == ref.view(np.uint32).tolist()


# ---- 3. exact-tile dispatch shapes --------------------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(16, 16, 16), (16, 48, 16), (32, 48, 32), (48, 16, 80),
                                   (128, 144, 272), (512, 256, 1024)])
def test_tiled_v1_dispatch_bit_exact_on_pinned_alphabet(gpu, oracle, m, n, k):
    a, b = oracle.generate_inputs_v1(m, n, k, m * 7 + n * 3 + k)
    assert oracle.validate_evidence_inputs_v1(m, n, k, a, b)[0] == 0
    gc = Guarded(gpu, np.full(m * n, np.nan, np.float32))
    _k().tiled_gemm_v1_gpu.Kernel.load(gpu).prepare(
        gpu.to_device(a), gpu.to_device(b), gc.body, m, n, k).launch()
    assert gc.guards_intact()
    rc, ref = oracle.tiled_gemm_arithmetic_v1(m, n, k, a, b)
    assert rc == 0
    assert gc.download().view(np.uint32).tolist() == ref.view(np.uint32).tolist()


@pytest.mark.parametrize("m,n,k", [(64, 80, 48), (256, 256, 512)])
def test_tiled_v1_dispatch_normal_inputs(gpu, oracle, m, n, k):
    rng = np.random.default_rng(m + n + k)
    a = oracle.bf16_from_f32(rng.standard_normal(m * k))
    b = oracle.bf16_from_f32(rng.standard_normal(k * n))
    gc = Guarded(gpu, np.full(m * n, np.nan, np.float32))
    _k().tiled_gemm_v1_gpu.Kernel.load(gpu).prepare(
        gpu.to_device(a), gpu.to_device(b), gc.body, m, n, k).launch()
    assert gc.guards_intact()
    rc, ref = oracle.tiled_gemm_arithmetic_v1(m, n, k, a, b)
    assert rc == 0
    assert rel_err(gc.download(), ref) <= 1e-5
