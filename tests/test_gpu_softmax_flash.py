"""GPU parity tests for row softmax and flash attention, through the C-ABI,
against the CPU oracle restatements.

Row softmax uses the reference's own comparison policy
(examples/row_softmax_v1/src/numerical_contract.rs:7-13: abs 3e-6 + rel
3e-5 or <= 64 ULP, active sum within 6e-5, masked outputs +0 bit-exact).
Flash attention: the exact f32 profile within 1e-5 (fp32 bar) of the
reference's two-pass f64 oracle; the bf16 BASELINE shape within rel-err
1e-2 of the same f64 oracle, plus the closed-form and invariance properties
of examples/flash_attention_v1/tests/oracle.rs.
"""
from __future__ import annotations

import numpy as np
import pytest

from golden import reference_vectors as rv
from gpu_util import Guarded, bf16_to_f32, rel_err

pytestmark = pytest.mark.gpu


def _k():
    from fe2o3_amd import kernels
    return kernels


# ---- row softmax ---------------------------------------------------------------------

def _softmax_v1(gpu, x):
    gi = Guarded(gpu, np.asarray(x, np.float32))
    go = Guarded(gpu, np.full(64, np.nan, np.float32))
    _k().row_softmax_v1_gpu.Kernel.load(gpu).prepare(gi.body, go.body).launch()
    assert gi.unchanged() and go.guards_intact()
    return go.download()


@pytest.mark.parametrize("idx", range(5))
def test_row_softmax_v1_corpus(gpu, oracle, idx):
    """tests/numerical_contract.rs:66-94 corpus under the OCML policy."""
    x = rv.softmax_corpus_v1()[idx]
    got = _softmax_v1(gpu, x)
    rc, ref, _ = oracle.row_softmax_oracle_v1(x)
    assert rc == 0
    rc, bad = oracle.compare_row_softmax_v1(ref, got, **oracle.GFX_SOFTMAX_POLICY)
    assert rc == 0, (rc, bad)


def test_row_softmax_v1_equal_row_is_exact(gpu):
    """numerical_contract.rs:105-111: an equal row gives exactly 1/64 each."""
    for x in (rv.softmax_corpus_v1()[0], rv.softmax_production_cases_v1()["equal"]):
        got = _softmax_v1(gpu, x)
        assert got.tolist() == [1.0 / 64.0] * 64


@pytest.mark.parametrize("name", ["normal", "equal", "dominant"])
def test_row_softmax_v1_production_cases(gpu, oracle, name):
    x = rv.softmax_production_cases_v1()[name]
    got = _softmax_v1(gpu, x)
    rc, ref, _ = oracle.row_softmax_oracle_v1(x)
    assert rc == 0
    assert oracle.compare_row_softmax_v1(ref, got, **oracle.GFX_SOFTMAX_POLICY)[0] == 0


@pytest.mark.parametrize("rows,cols,masked", [(7, 64, False), (33, 100, True), (64, 256, True),
                                              (129, 4096, False), (40, 4096, True),
                                              (9, 5000, True), (5, 8192, False)])
def test_row_softmax_rows_against_oracle(gpu, oracle, rows, cols, masked):
    rng = np.random.default_rng(rows * 131 + cols)
    x = (rng.standard_normal(rows * cols) * 4.0).astype(np.float32)
    mask = None
    if masked:
        mask = (rng.random(rows * cols) < 0.8).astype(np.uint8)
        mask[:cols] = 0  # first row fully masked -> all +0
    gi = Guarded(gpu, x)
    go = Guarded(gpu, np.full(rows * cols, np.nan, np.float32))
    gm = Guarded(gpu, mask) if masked else None
    _k().row_softmax_gpu.Kernel.load(gpu).prepare(
        gi.body, go.body, gm.body if masked else None, rows, cols).launch()
    got = go.download().reshape(rows, cols)
    assert go.guards_intact() and gi.unchanged()
    for r in range(rows):
        m = None if mask is None else mask[r * cols:(r + 1) * cols]
        if m is not None and m.sum() == 0:
            assert got[r].view(np.uint32).tolist() == [0] * cols
            continue
        xr = x[r * cols:(r + 1) * cols]
        if cols <= 4096:
            rc, ref, _ = oracle.row_softmax_oracle_v1(xr, m)
            assert rc == 0
        else:
            # the reference oracle refuses rows above 4096 elements
            # (examples/row_softmax_v1/src/numerical_contract.rs:4); wider rows
            # are checked against a float64 evaluation of the same formula
            act = np.ones(cols, bool) if m is None else m.astype(bool)
            w = np.where(act, np.exp(xr.astype(np.float64) - xr[act].max()), 0.0)
            ref = (w / w.sum()).astype(np.float32)
        rc, bad = oracle.compare_row_softmax_v1(ref, got[r], m, **oracle.GFX_SOFTMAX_POLICY)
        assert rc == 0, (r, rc, bad)


def test_row_softmax_config3c_every_row(gpu, oracle):
    """BASELINE config 3c at full size: 1,048,576 rows x 4096 fp32 (the
    bench's N(0,1) input, seed 3).  Every row, element by element, against
    the f64 oracle under the OCML comparison policy (abs 3e-6 + rel 3e-5 or
    64 ULP per element, row sum within 6e-5), checked in C over the rows of
    each 1 GiB chunk (oracle.row_softmax_check_rows)."""
    rows, cols = 8 * 32 * 4096, 4096
    kern = _k()
    x = gpu.alloc(rows * cols, np.float32)
    kern.fill_normal_f32(x, 3, 0x50F7, 1.0)
    y = gpu.alloc(rows * cols, np.float32)
    kern.row_softmax_gpu.Kernel.load(gpu).prepare(x, y, None, rows, cols).launch()
    chunk = 65536
    checked = 0
    for c0 in range(0, rows, chunk):
        hx = x.view(c0 * cols, chunk * cols).download()
        hy = y.view(c0 * cols, chunk * cols).download()
        rc, st = oracle.row_softmax_check_rows(hx, hy, chunk, cols, **oracle.GFX_SOFTMAX_POLICY)
        assert rc == 0, (c0, rc)
        assert st["failing_rows"] == 0, (c0 + st["first_failing_row"], st)
        assert st["max_row_sum_err"] <= 6e-5, (c0, st)
        checked += chunk
    assert checked == rows


def test_row_softmax_rejects_zero_cols(gpu):
    from fe2o3_amd.runtime import Fe2o3Error
    a = gpu.alloc(4, np.float32)
    with pytest.raises(Fe2o3Error) as e:
        _k().row_softmax_gpu.Kernel.load(gpu).prepare(a, a, None, 4, 0).launch()
    assert e.value.status == -3


# ---- flash attention: exact profile ---------------------------------------------------------

def _flash_profile(gpu, q, k, v):
    bufs = [Guarded(gpu, np.asarray(t, np.float32)) for t in (q, k, v)]
    go = Guarded(gpu, np.full(128, np.nan, np.float32))
    _k().flash_attention_causal_f32_b1_h1_n8_d16_v1_gpu.Kernel.load(gpu).prepare(
        bufs[0].body, bufs[1].body, bufs[2].body, go.body).launch()
    assert all(b.unchanged() for b in bufs) and go.guards_intact()
    return go.download()


@pytest.mark.parametrize("which", ["reference_vectors", "hardware_vectors"])
def test_flash_profile_against_f64_oracle(gpu, oracle, which):
    vecs = rv.flash_vectors_v1() if which == "reference_vectors" else rv.flash_hardware_vectors_v1()
    for name, q, k, v in vecs:
        got = _flash_profile(gpu, q, k, v)
        rc, ref, _, _ = oracle.flash_attention_v1(q, k, v)
        assert rc == 0, name
        assert np.all(np.abs(got - ref) <= 1e-5 * np.maximum(1.0, np.abs(ref))), name
        assert rel_err(got, ref) <= 1e-5, name


def test_flash_profile_closed_forms(gpu):
    """examples/flash_attention_v1/tests/oracle.rs:44-73: equal logits give the
    causal prefix means of V; a dominant latest key returns its V row."""
    name, q, k, v = rv.flash_vectors_v1()[1]  # all-equal-logits
    got = _flash_profile(gpu, q, k, v).reshape(8, 16)
    vv = v.reshape(8, 16).astype(np.float64)
    for r in range(8):
        assert np.allclose(got[r], vv[:r + 1].mean(axis=0), rtol=0, atol=1e-6)
    name, q, k, v = rv.flash_vectors_v1()[2]  # latest-causal-key-dominates
    got = _flash_profile(gpu, q, k, v).reshape(8, 16)
    for r in range(8):
        assert np.all(np.abs(got[r] - v.reshape(8, 16)[r]) <= 1e-5)


# ---- flash attention: BASELINE shape -----------------------------------------------------------

def _flash(gpu, b, h, s, causal, seed, lse=True, qkv=None):
    kern = _k()
    n = b * h * s * 128
    scale = 1.0 / np.sqrt(128.0)
    if qkv is None:
        bufs = [gpu.alloc(n, np.uint16) for _ in range(3)]
        for i, t in enumerate(bufs):
            kern.fill_normal_bf16(t, seed, 0xF100 + i, 1.0)
    else:
        bufs = [gpu.to_device(t) for t in qkv]
    o = Guarded(gpu, np.full(n, 0x7FDE, np.uint16))
    l = Guarded(gpu, np.full(b * h * s, np.nan, np.float32)) if lse else None
    kern.flash_attention_fwd_gpu.Kernel.load(gpu).prepare(
        bufs[0], bufs[1], bufs[2], o.body, l.body if lse else None, b, h, s, 128,
        1 if causal else 0, scale).launch()
    assert o.guards_intact() and (l is None or l.guards_intact())
    host = [t.download() for t in bufs]
    return host, bf16_to_f32(o.download()), (l.download() if lse else None), scale


@pytest.mark.parametrize("causal", [False, True])
# causal: an even query-tile count (256, 512) pairs tiles per workgroup; an
# odd one (128, 384) runs one tile per workgroup
@pytest.mark.parametrize("b,h,s", [(1, 1, 128), (1, 2, 256), (1, 1, 384), (2, 1, 512)])
def test_flash_small_all_rows(gpu, oracle, b, h, s, causal):
    (q, k, v), out, lse, scale = _flash(gpu, b, h, s, causal, seed=2)
    bh = np.repeat(np.arange(b * h, dtype=np.uint32), s)
    rows = np.tile(np.arange(s, dtype=np.uint32), b * h)
    rc, ref, ref_lse = oracle.flash_attention_rows_bf16(q, k, v, s, 128, causal, scale, bh, rows)
    assert rc == 0
    got = out.reshape(-1, 128)
    assert rel_err(got, ref) <= 1e-2
    assert rel_err(lse, ref_lse) <= 1e-5  # fp32 output: the 1e-5 bar


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("pattern", ["ramp", "spikes", "jump"])
def test_flash_rescales_all_rows(gpu, oracle, pattern, causal):
    """Scores that force the running reference up again and again: every key
    tile raises every row's max by ~16 (log2 units; ramp), random keys far
    above the rest (spikes), or a jump of ~228 halfway, where the
    exponentials against the old reference overflow to +inf (jump).  Every
    row and its LSE against the f64 oracle."""
    b, h, s = 1, 2, 512
    rng = np.random.default_rng({"ramp": 1, "spikes": 2, "jump": 3}[pattern])
    t = np.zeros(b * h * s, np.float32)
    j = np.tile(np.arange(s), b * h)
    if pattern == "ramp":
        t = (j / 64.0).astype(np.float32)
    elif pattern == "spikes":
        t = np.where(rng.random(b * h * s) < 0.04, 6.0, 0.0).astype(np.float32)
    else:
        t = np.where(j >= s // 2, 14.0, 0.0).astype(np.float32)
    q = np.ones((b * h * s, 128), np.float32) + 0.05 * rng.standard_normal((b * h * s, 128))
    k = t[:, None] + 0.1 * rng.standard_normal((b * h * s, 128))
    v = rng.standard_normal((b * h * s, 128))
    qkv = [oracle.bf16_from_f32(np.ascontiguousarray(x, np.float32).ravel()) for x in (q, k, v)]
    (qh, kh, vh), out, lse, scale = _flash(gpu, b, h, s, causal, seed=0, qkv=qkv)
    bh = np.repeat(np.arange(b * h, dtype=np.uint32), s)
    rows = np.tile(np.arange(s, dtype=np.uint32), b * h)
    rc, ref, ref_lse = oracle.flash_attention_rows_bf16(qh, kh, vh, s, 128, causal, scale, bh, rows)
    assert rc == 0
    assert np.all(np.isfinite(out)) and np.all(np.isfinite(lse))
    assert rel_err(out.reshape(-1, 128), ref) <= 1e-2
    assert rel_err(lse, ref_lse) <= 1e-5  # fp32 output: the 1e-5 bar


@pytest.mark.parametrize("causal", [False, True])
def test_flash_config3_sampled_rows(gpu, oracle, causal):
    """B8 H32 S4096 D128, Q/K/V ~ N(0,1) bf16, scale
    1/sqrt(128), against the two-pass f64 oracle with the LSE: 64 query rows
    in every one of the 256 (batch, head), one per 64-row band at a position
    that varies with the head and band (16,384 rows), plus 64 rows (first,
    last and 128-row tile edges among them) in 16 heads spread over every
    batch."""
    b, h, s = 8, 32, 4096
    (q, k, v), out, lse, scale = _flash(gpu, b, h, s, causal, seed=2)
    per = 64
    bh_all = np.repeat(np.arange(b * h, dtype=np.uint32), per)
    band = np.tile(np.arange(per, dtype=np.uint32), b * h)
    rows_all = band * (s // per) + (bh_all * 67 + band * 131) % (s // per)
    heads = [i * 16 + (i * 5) % 16 for i in range(16)]
    qrows = sorted({0, 1, 127, 128, 2047, 2048, 4094, 4095} |
                   {int(r) for r in np.random.default_rng(3).integers(0, s, 56)})
    qrows = (qrows + [255, 256, 383, 384, 511, 512, 3967, 3968])[:64]
    bh = np.concatenate([bh_all, np.array([hh for hh in heads for _ in qrows], np.uint32)])
    rows = np.concatenate([rows_all, np.array(qrows * len(heads), np.uint32)]).astype(np.uint32)
    rc, ref, ref_lse = oracle.flash_attention_rows_bf16(q, k, v, s, 128, causal, scale, bh, rows)
    assert rc == 0
    got = out.reshape(b * h, s, 128)[bh, rows]
    assert rel_err(got, ref) <= 1e-2
    assert rel_err(lse.reshape(b * h, s)[bh, rows], ref_lse) <= 1e-5  # fp32 output: the 1e-5 bar


def test_flash_causal_ignores_future_keys(gpu):
    """examples/flash_attention_v1/tests/oracle.rs:75-96: causal rows q < s/2
    are bit-identical when keys/values beyond s/2 change."""
    b, h, s = 1, 1, 512
    (q, k, v), out1, _, _ = _flash(gpu, b, h, s, True, seed=9)
    k2, v2 = k.copy(), v.copy()
    rng = np.random.default_rng(0)
    k2[(s // 2) * 128:] = rng.integers(0x3C00, 0x4000, size=k2[(s // 2) * 128:].size, dtype=np.uint16)
    v2[(s // 2) * 128:] = rng.integers(0x3C00, 0x4000, size=v2[(s // 2) * 128:].size, dtype=np.uint16)
    _, out2, _, _ = _flash(gpu, b, h, s, True, seed=0, qkv=(q, k2, v2))
    half = (s // 2) * 128
    assert out1[:half].tobytes() == out2[:half].tobytes()
    assert out1[half:].tobytes() != out2[half:].tobytes()


def test_flash_noncausal_key_permutation_invariance(gpu):
    b, h, s = 1, 1, 256
    (q, k, v), out1, _, _ = _flash(gpu, b, h, s, False, seed=4)
    perm = np.random.default_rng(1).permutation(s)
    k2 = k.reshape(s, 128)[perm].ravel()
    v2 = v.reshape(s, 128)[perm].ravel()
    _, out2, _, _ = _flash(gpu, b, h, s, False, seed=0, qkv=(q, k2, v2))
    assert rel_err(out2, out1) <= 1e-2


def test_flash_rejects_bad_shapes(gpu):
    """head_dim other than 128 and a scale that is not positive and finite
    are refused before any launch, the output untouched."""
    from fe2o3_amd.runtime import Fe2o3Error
    a = gpu.alloc(100 * 64, np.uint16)
    K = _k().flash_attention_fwd_gpu.Kernel.load(gpu)
    with pytest.raises(Fe2o3Error) as e:
        K.prepare(a, a, a, a, None, 1, 1, 100, 64, 0, 0.125).launch()
    assert e.value.status == -3
    b = gpu.to_device(np.zeros(100 * 128, np.uint16))
    o = Guarded(gpu, np.full(100 * 128, 0x7FDE, np.uint16))
    for bad in (0.0, -0.125, float("inf"), float("nan")):
        with pytest.raises(Fe2o3Error) as e:
            K.prepare(b, b, b, o.body, None, 1, 1, 100, 128, 0, bad).launch()
        assert e.value.status == -3
    assert o.unchanged()


def _guarded_qkv(gpu, b, h, s, seed):
    """Q, K, V ~ N(0,1) bf16 in guard-banded buffers (bf16 NaN guards): a
    read past a head's seq rows of the last (batch, head) would meet NaN."""
    rng = np.random.default_rng(seed)
    n = b * h * s * 128
    host = [(rng.standard_normal(n).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
            for _ in range(3)]
    return host, [Guarded(gpu, t) for t in host]


@pytest.mark.parametrize("causal", [False, True])
# partial last query tiles (seq % 128) and key tiles (seq % 64), one key
# tile only (1, 37, 64), odd and even query-tile counts (causal pairing)
@pytest.mark.parametrize("b,h,s", [(1, 1, 1), (1, 2, 37), (1, 1, 64), (2, 1, 100), (1, 1, 129),
                                   (1, 2, 200), (1, 1, 1000)])
def test_flash_any_seq_all_rows(gpu, oracle, b, h, s, causal):
    """seq not a multiple of 128: every row and its LSE against the f64
    oracle; outputs past seq untouched (guards), inputs unchanged."""
    host, (gq, gk, gv) = _guarded_qkv(gpu, b, h, s, seed=s + 7 * b + h)
    n = b * h * s * 128
    scale = 1.0 / np.sqrt(128.0)
    o = Guarded(gpu, np.full(n, 0x7FDE, np.uint16))
    l = Guarded(gpu, np.full(b * h * s, np.nan, np.float32))
    _k().flash_attention_fwd_gpu.Kernel.load(gpu).prepare(
        gq.body, gk.body, gv.body, o.body, l.body, b, h, s, 128, 1 if causal else 0,
        scale).launch()
    assert o.guards_intact() and l.guards_intact()
    assert gq.unchanged() and gk.unchanged() and gv.unchanged()
    bh = np.repeat(np.arange(b * h, dtype=np.uint32), s)
    rows = np.tile(np.arange(s, dtype=np.uint32), b * h)
    rc, ref, ref_lse = oracle.flash_attention_rows_bf16(*host, s, 128, causal, scale, bh, rows)
    assert rc == 0
    got = bf16_to_f32(o.download()).reshape(-1, 128)
    assert np.all(np.isfinite(got))
    assert rel_err(got, ref) <= 1e-2
    assert rel_err(l.download(), ref_lse) <= 1e-5  # fp32 output: the 1e-5 bar


def test_flash_partial_key_tile_ignores_stale_lds(gpu, oracle):
    """The rows of a partial key tile past seq are read as zero, not left
    as they were: a launch whose V is all NaN (seq 64, 512 heads, every CU
    busy) leaves NaN rows in LDS, and a following launch at seq 37 still
    matches the oracle with finite outputs."""
    kern = _k().flash_attention_fwd_gpu.Kernel.load(gpu)
    heads, s0 = 512, 64
    n0 = heads * s0 * 128
    q0 = gpu.to_device(np.full(n0, 0x3F80, np.uint16))  # 1.0
    v0 = gpu.to_device(np.full(n0, 0x7FC0, np.uint16))  # NaN
    o0 = gpu.alloc(n0, np.uint16)
    kern.prepare(q0, q0, v0, o0, None, 1, heads, s0, 128, 0, 0.125).launch()
    for causal in (False, True):
        b, h, s = 1, 64, 37
        host, (gq, gk, gv) = _guarded_qkv(gpu, b, h, s, seed=11)
        n = b * h * s * 128
        o = Guarded(gpu, np.full(n, 0x7FDE, np.uint16))
        kern.prepare(gq.body, gk.body, gv.body, o.body, None, b, h, s, 128, int(causal),
                     0.125).launch()
        got = bf16_to_f32(o.download()).reshape(-1, 128)
        assert np.all(np.isfinite(got)) and o.guards_intact()
        bh = np.repeat(np.arange(b * h, dtype=np.uint32), s)
        rows = np.tile(np.arange(s, dtype=np.uint32), b * h)
        rc, ref, _ = oracle.flash_attention_rows_bf16(*host, s, 128, causal, 0.125, bh, rows)
        assert rc == 0
        assert rel_err(got, ref) <= 1e-2
