"""The protected profile lifecycles (fe2o3_protected_*) through the library's
HIP adapter on the GPU: each profile's embedded code object is loaded,
resolved, dispatched with its explicit kernarg and the implicit suffix the
adapter writes, and unloaded; the outputs are judged against the CPU oracle
as the library entry points are (tests/test_gpu_softmax_flash.py,
tests/test_gpu_moe_fp8.py).  Each code object runs the routine the library's
own profile entry runs (profiles.hpp), so the flash and routing outputs are
also compared bit for bit with the library entry points'.

crates/fe2o3-host/src/flash_attention_v1_lifecycle.rs,
protected_row_softmax_v1_lifecycle.rs, moe_top2_v1_lifecycle.rs.
"""
from __future__ import annotations

import numpy as np
import pytest

from golden import reference_vectors as rv
from gpu_util import Guarded, rel_err

pytestmark = pytest.mark.gpu

ROUTE_KEYS = ["top2_experts", "requested_counts", "admitted_counts", "expert_offsets",
              "route_slots", "permutation", "inverse"]
ROUTE_LENS = [16, 4, 4, 5, 16, 16, 16]


class Leases:
    def __init__(self):
        self.drops = 0

    def __call__(self):
        self.drops += 1


def _run(joined):
    """load (HIP adapter) -> dispatch_and_wait -> unload; the receipt."""
    completed = joined.load().dispatch_and_wait()
    receipt = completed.unload()
    assert receipt.identity == joined.identity
    assert receipt.artifact_identity == joined.artifact_identity
    return receipt


def _flash_lifecycle(gpu, q, k, v):
    from fe2o3_amd import lifecycle as lc
    bufs = [Guarded(gpu, np.asarray(x, np.float32)) for x in (q, k, v)]
    out = Guarded(gpu, np.full(128, np.nan, np.float32))
    leases = Leases()
    _run(lc.join_flash_attention_v1(bufs[0].body, bufs[1].body, bufs[2].body, out.body,
                                    on_release=leases))
    assert leases.drops == 1
    assert all(b.unchanged() for b in bufs) and out.guards_intact()
    return out.download()


def _flash_entry(gpu, q, k, v):
    from fe2o3_amd import kernels
    bufs = [gpu.to_device(np.asarray(x, np.float32)) for x in (q, k, v)]
    out = gpu.alloc(128, np.float32)
    kernels.flash_attention_causal_f32_b1_h1_n8_d16_v1_gpu.Kernel.load(gpu).prepare(
        *bufs, out).launch()
    return out.download()


@pytest.mark.parametrize("which", ["reference_vectors", "hardware_vectors"])
def test_flash_lifecycle_against_oracle_and_entry_point(gpu, oracle, which):
    vecs = rv.flash_vectors_v1() if which == "reference_vectors" else rv.flash_hardware_vectors_v1()
    for name, q, k, v in vecs:
        got = _flash_lifecycle(gpu, q, k, v)
        rc, ref, _, _ = oracle.flash_attention_v1(q, k, v)
        assert rc == 0, name
        assert np.all(np.abs(got - ref) <= 1e-5 * np.maximum(1.0, np.abs(ref))), name
        assert rel_err(got, ref) <= 1e-5, name
        assert got.view(np.uint32).tolist() == _flash_entry(gpu, q, k, v).view(np.uint32).tolist()


def _softmax_lifecycle(gpu, x):
    from fe2o3_amd import lifecycle as lc
    gx = Guarded(gpu, np.asarray(x, np.float32))
    gy = Guarded(gpu, np.full(64, np.nan, np.float32))
    _run(lc.join_row_softmax_v1(gx.body, gy.body))
    assert gx.unchanged() and gy.guards_intact()
    return gy.download()


def test_row_softmax_lifecycle_corpus_and_production_cases(gpu, oracle):
    """tests/numerical_contract.rs:66-94 corpus and the production cases
    under the OCML policy; an equal row gives exactly 1/64."""
    production = rv.softmax_production_cases_v1()
    cases = list(rv.softmax_corpus_v1()) + [production[k] for k in ("normal", "equal", "dominant")]
    for x in cases:
        got = _softmax_lifecycle(gpu, x)
        rc, ref, _ = oracle.row_softmax_oracle_v1(x)
        assert rc == 0
        rc, bad = oracle.compare_row_softmax_v1(ref, got, **oracle.GFX_SOFTMAX_POLICY)
        assert rc == 0, (rc, bad)
    assert _softmax_lifecycle(gpu, rv.softmax_production_cases_v1()["equal"]).tolist() == \
        [1.0 / 64.0] * 64


@pytest.mark.parametrize("name", list(rv.MOE_VECTORS))
def test_moe_top2_lifecycle_bit_exact(gpu, oracle, name):
    """examples/moe_top2_v1/src/vectors.rs:14-117: every routing array
    bit-equal to the oracle and to the library's entry point."""
    from fe2o3_amd import kernels
    from fe2o3_amd import lifecycle as lc
    logits = np.array(rv.MOE_VECTORS[name], np.float32)
    rc, ref = oracle.moe_top2_route(logits, 8, 4, 4)
    assert rc == 0
    gl = Guarded(gpu, logits)
    outs = [Guarded(gpu, np.full(n, 0xABABABAB, np.uint32)) for n in ROUTE_LENS]
    _run(lc.join_moe_top2_v1(gl.body, *[o.body for o in outs]))
    assert gl.unchanged()
    entry = [gpu.alloc(n, np.uint32) for n in ROUTE_LENS]
    kernels.moe_top2_route_f32_t8_e4_k2_c4_v1_gpu.Kernel.load(gpu).prepare(
        gpu.to_device(logits), *entry).launch()
    for key, o, e in zip(ROUTE_KEYS, outs, entry):
        assert o.guards_intact(), key
        got = o.download().tolist()
        assert got == ref[key].tolist(), key
        assert got == e.download().tolist(), key


def test_protected_lifecycle_observations_on_the_device(gpu):
    """The HIP adapter's observations pass every load check for each profile:
    the resolved kernarg segment is the profile's complete ABI, no static LDS,
    no private segment; a second load of the same profile gets other object
    identities."""
    from fe2o3_amd import lifecycle as lc
    for profile, n in ((lc.FLASH_ATTENTION_V1, [128] * 4), (lc.ROW_SOFTMAX_V1, [64, 64]),
                       (lc.MOE_TOP2_V1, [32] + ROUTE_LENS)):
        prof = lc.protected_profile(profile)
        seen = set()
        for _ in range(2):
            bufs = [gpu.alloc(e, np.float32) for e in n]
            loaded = lc.join_protected_v1(profile, bufs).load()
            o = loaded.observation()
            assert o.resolution.symbol == prof.symbol
            assert o.resolution.kernarg_segment_bytes == prof.complete_kernarg_bytes
            assert o.resolution.kernarg_alignment >= 16
            assert (o.resources.group_segment_bytes, o.resources.private_segment_bytes) == (0, 0)
            seen.add(bytes(o.load.executable_object))
            loaded.release()
        assert len(seen) == 2
