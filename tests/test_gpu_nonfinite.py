"""Fail-closed handling of non-finite inputs, through the C-ABI.

The reference's router and flash-attention profile trap on any NaN or
infinite input (examples/moe_top2_v1/src/kernel.rs:118-128,
examples/flash_attention_v1/src/kernel.rs:137-146) and its row-softmax
contract rejects a row holding one, masked elements included
(examples/row_softmax_v1/src/numerical_contract.rs:145-151).  Here the
kernels write their documented sentinels, mark the device's contract-status
word and exit normally; the synchronizing launch then raises
FE2O3_ERR_NONFINITE (-5).  Each case checks that status, the sentinel
outputs, intact guards and unchanged inputs, that the CPU oracle rejects the
same input with the same code, and that the status is cleared afterwards (a
following clean launch succeeds).
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import Guarded

pytestmark = pytest.mark.gpu

BAD = {"nan": np.float32(np.nan), "+inf": np.float32(np.inf), "-inf": np.float32(-np.inf)}
QNAN = 0x7FC00000
DROP = 0xFFFFFFFF


def _k():
    from fe2o3_amd import kernels
    return kernels


def _expect_nonfinite(fn):
    from fe2o3_amd.runtime import Fe2o3Error
    with pytest.raises(Fe2o3Error) as ei:
        fn()
    assert ei.value.status == -5, ei.value


# ---- row softmax ------------------------------------------------------------------------

@pytest.mark.parametrize("bad", list(BAD))
def test_row_softmax_v1_rejects(gpu, oracle, bad):
    x = np.linspace(-3, 3, 64).astype(np.float32)
    x[17] = BAD[bad]
    assert oracle.row_softmax_oracle_v1(x)[0] == -5
    gi = Guarded(gpu, x)
    go = Guarded(gpu, np.zeros(64, np.float32))
    prep = _k().row_softmax_v1_gpu.Kernel.load(gpu).prepare(gi.body, go.body)
    _expect_nonfinite(prep.launch)
    assert gi.unchanged() and go.guards_intact()
    assert go.download().view(np.uint32).tolist() == [QNAN] * 64
    # the status was taken: a clean row now launches without error
    gi2 = Guarded(gpu, np.zeros(64, np.float32))
    _k().row_softmax_v1_gpu.Kernel.load(gpu).prepare(gi2.body, go.body).launch()
    assert go.download().tolist() == [1.0 / 64.0] * 64


@pytest.mark.parametrize("cols,masked", [(4096, False), (4096, True), (100, False), (100, True),
                                         (256, True)])
def test_row_softmax_rejects_only_bad_rows(gpu, oracle, cols, masked):
    """Rows 1 (NaN), 4 (+inf) and 6 (-inf, masked out when a mask is used)
    are rejected; the other rows match the oracle under the OCML policy."""
    rows = 8
    rng = np.random.default_rng(cols + masked)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    mask = (rng.random((rows, cols)) < 0.7).astype(np.uint8) if masked else None
    x[1, 5], x[4, cols - 1], x[6, cols // 2] = np.nan, np.inf, -np.inf
    if masked:
        mask[6, cols // 2] = 0  # masked, still rejected (the contract checks every element)
    bad_rows = {1, 4, 6}
    gi = Guarded(gpu, x)
    go = Guarded(gpu, np.zeros(rows * cols, np.float32))
    gm = Guarded(gpu, mask) if masked else None
    prep = _k().row_softmax_gpu.Kernel.load(gpu).prepare(
        gi.body, go.body, gm.body if masked else None, rows, cols)
    _expect_nonfinite(prep.launch)
    assert gi.unchanged() and go.guards_intact()
    got = go.download().reshape(rows, cols)
    for r in range(rows):
        m = None if mask is None else mask[r]
        if r in bad_rows:
            assert oracle.row_softmax_oracle_v1(x[r], m)[0] == -5
            assert got[r].view(np.uint32).tolist() == [QNAN] * cols, r
            continue
        rc, ref, _ = oracle.row_softmax_oracle_v1(x[r], m)
        assert rc == 0
        assert oracle.compare_row_softmax_v1(ref, got[r], m, **oracle.GFX_SOFTMAX_POLICY)[0] == 0
    # finite rows alone: no status
    x[[1, 4, 6]] = 0.0
    gi2 = Guarded(gpu, x)
    _k().row_softmax_gpu.Kernel.load(gpu).prepare(
        gi2.body, go.body, gm.body if masked else None, rows, cols).launch()


# ---- flash attention exact profile -------------------------------------------------------

@pytest.mark.parametrize("where", ["q", "k", "v"])
@pytest.mark.parametrize("bad", list(BAD))
def test_flash_profile_rejects(gpu, oracle, where, bad):
    rng = np.random.default_rng(3)
    qkv = {n: rng.standard_normal(128).astype(np.float32) for n in "qkv"}
    qkv[where][77] = BAD[bad]
    assert oracle.flash_attention_v1(qkv["q"], qkv["k"], qkv["v"])[0] == -5
    g = {n: Guarded(gpu, qkv[n]) for n in "qkv"}
    go = Guarded(gpu, np.zeros(128, np.float32))
    prep = _k().flash_attention_causal_f32_b1_h1_n8_d16_v1_gpu.Kernel.load(gpu).prepare(
        g["q"].body, g["k"].body, g["v"].body, go.body)
    _expect_nonfinite(prep.launch)
    assert all(g[n].unchanged() for n in "qkv") and go.guards_intact()
    assert go.download().view(np.uint32).tolist() == [QNAN] * 128


# ---- top-2 router --------------------------------------------------------------------------

ROUTE_KEYS = ["top2_experts", "requested_counts", "admitted_counts", "expert_offsets",
              "route_slots", "permutation", "inverse"]


@pytest.mark.parametrize("bad", list(BAD))
def test_route_profile_rejects(gpu, oracle, bad):
    logits = np.random.default_rng(4).standard_normal(32).astype(np.float32)
    logits[13] = BAD[bad]
    assert oracle.moe_top2_route(logits, 8, 4, 4)[0] == -5
    lens = [16, 4, 4, 5, 16, 16, 16]
    outs = [Guarded(gpu, np.full(n, 0xABABABAB, np.uint32)) for n in lens]
    gl = Guarded(gpu, logits)
    prep = _k().moe_top2_route_f32_t8_e4_k2_c4_v1_gpu.Kernel.load(gpu).prepare(
        gl.body, *[o.body for o in outs])
    _expect_nonfinite(prep.launch)
    assert gl.unchanged()
    got = {key: o.download().tolist() for key, o in zip(ROUTE_KEYS, outs)}
    assert all(o.guards_intact() for o in outs)
    assert got["top2_experts"] == [DROP] * 16
    assert got["requested_counts"] == [0] * 4 and got["admitted_counts"] == [0] * 4
    assert got["expert_offsets"] == [0] * 5
    for key in ("route_slots", "permutation", "inverse"):
        assert got[key] == [DROP] * 16, key


@pytest.mark.parametrize("tokens", [4096, 20000])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("bad", list(BAD))
def test_route_rejects_whole_launch(gpu, oracle, dtype, bad, tokens):
    """One non-finite logit among `tokens` tokens x 8 experts rejects the
    launch: every output is its sentinel, weights +0, and a following FFN
    over that routing writes an all-zero output (no expert receives a
    route).  20000 tokens take the count / scan / assign kernels, with the
    bad token in the last workgroup."""
    experts = 8
    rng = np.random.default_rng(9)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    logits[3001 if tokens == 4096 else tokens - 7, 5] = BAD[bad]
    assert oracle.moe_top2_route(logits, tokens, experts)[0] == -5
    if dtype == "bf16":
        dev = gpu.to_device(oracle.bf16_from_f32(logits.ravel()))
    else:
        dev = gpu.to_device(logits.ravel())
    n = 2 * tokens
    out = {"top2": gpu.alloc(n, np.uint32), "requested": gpu.alloc(experts, np.uint32),
           "admitted": gpu.alloc(experts, np.uint32), "offsets": gpu.alloc(experts + 1, np.uint32),
           "slots": gpu.alloc(n, np.uint32), "permutation": gpu.alloc(n, np.uint32),
           "inverse": gpu.alloc(n, np.uint32), "weights": gpu.alloc(n, np.float32)}
    _expect_nonfinite(lambda: _k().moe_top2_route(dev, out, tokens, experts))
    for key in ("top2", "slots", "permutation", "inverse"):
        assert np.all(out[key].download() == DROP), key
    for key in ("requested", "admitted", "offsets"):
        assert np.all(out[key].download() == 0), key
    assert out["weights"].download().view(np.uint32).tolist() == [0] * n
    # the FFN over a rejected routing: no route admitted, output all +0
    hidden, ffn = 256, 256
    x = gpu.to_device(oracle.bf16_from_f32(rng.standard_normal(tokens * hidden)))
    w = [gpu.to_device(oracle.bf16_from_f32(rng.standard_normal(experts * ffn * hidden) * 0.02))
         for _ in range(3)]
    y = Guarded(gpu, np.full(tokens * hidden, 0x7FDE, np.uint16))
    ws = gpu.alloc(_k().moe_ffn_workspace_bytes(tokens, hidden, ffn, experts), np.uint8)
    _k().moe_ffn_top2(x, w[0], w[1], w[2], out, y.body, ws, tokens, hidden, ffn, experts)
    assert y.guards_intact()
    assert np.all(y.download() == 0)
