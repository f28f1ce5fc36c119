"""The exact LDS GEMM lifecycle on the GPU through the library's HIP adapter:
the embedded gfx950 code object is loaded from memory, resolved, observed,
dispatched once with its 304-byte kernarg (48 explicit bytes plus the
implicit suffix) and unloaded.  The product is judged like the library's
slice-1 entry point (tests/test_gpu_gemm.py: the reference's six-case
hardware matrix, crates/fe2o3-hsa-runtime/tests/tiled_gemm_lds_v1_hardware.rs:
778-979): exact cases bit for bit against the arithmetic oracle, the others
within 64*eps*sum|p| + FLT_MIN of the f64 product.  The kernel writes quiet
NaN instead of a product when the implicit suffix does not carry the
launch's block count and workgroup size, so a bit-exact C also shows the
implicit arguments were initialized.
"""
from __future__ import annotations

import numpy as np
import pytest

from golden import reference_vectors as rv
from gpu_util import Guarded

pytestmark = pytest.mark.gpu

FLT_EPS = np.float32(np.finfo(np.float32).eps)
FLT_MIN = np.float32(np.finfo(np.float32).tiny)


def _lc():
    from fe2o3_amd import lifecycle
    return lifecycle


class Leases:
    def __init__(self):
        self.drops = 0

    def __call__(self):
        self.drops += 1


def _check_product(oracle, a, b, got, exact):
    if exact:
        rc, ref = oracle.tiled_gemm_arithmetic_v1(16, 16, 16, a, b)
        assert rc == 0
        assert got.view(np.uint32).tolist() == ref.view(np.uint32).tolist()
    else:
        af = oracle.bf16_to_f32(a).astype(np.float64).reshape(16, 16)
        bf = oracle.bf16_to_f32(b).astype(np.float64).reshape(16, 16)
        bound = 64 * float(FLT_EPS) * (np.abs(af) @ np.abs(bf)) + float(FLT_MIN)
        assert np.all(np.isfinite(got))
        assert np.all(np.abs(got.reshape(16, 16) - af @ bf) <= bound)


@pytest.mark.parametrize("case", [c[0] for c in rv.lds_tile_cases()])
def test_lifecycle_six_cases(gpu, oracle, case):
    lc = _lc()
    _, a, b, exact = next(c for c in rv.lds_tile_cases() if c[0] == case)
    a = np.array(a, np.uint16)
    b = np.array(b, np.uint16)
    ga, gb = Guarded(gpu, a), Guarded(gpu, b)
    gc = Guarded(gpu, np.full(256, np.nan, np.float32))
    leases = Leases()
    loaded = lc.join_exact_lds_gemm_slice1_v1(ga.body, gb.body, gc.body,
                                              on_release=leases).load()
    completed = loaded.dispatch_and_wait()
    assert leases.drops == 1
    receipt = completed.unload()
    assert ga.unchanged() and gb.unchanged() and gc.guards_intact()
    _check_product(oracle, a, b, gc.download(), exact)
    art = lc.artifact()
    assert receipt.finalizer_identity == bytes(art.finalizer_identity)
    assert any(receipt.unload_identity)


def test_lifecycle_observations_on_the_device(gpu, oracle):
    """What the HIP adapter observes: a gfx950 target compatible with
    gfx950:xnack-, the caller's ordinal, the loaded bytes' digest and
    length, the 304-byte kernarg segment at 16-byte dispatch alignment, 1024
    bytes of static LDS and no private segment."""
    lc = _lc()
    rng = np.random.default_rng(5)
    a = oracle.bf16_from_f32(rng.integers(-8, 8, 256).astype(np.float32))
    b = oracle.bf16_from_f32(rng.integers(-8, 8, 256).astype(np.float32))
    ga, gb = gpu.to_device(a), gpu.to_device(b)
    gc = Guarded(gpu, np.full(256, np.nan, np.float32))
    loaded = lc.join_exact_lds_gemm_slice1_v1(ga, gb, gc.body).load()
    obs = loaded.observation()
    art = lc.artifact()
    assert obs.state == lc.LOADED and obs.holds_executable and obs.holds_kernel
    env = obs.environment
    assert env.physical_target.startswith(b"gfx950") and b"xnack+" not in env.physical_target
    assert env.hip_ordinal == 0 and bytes(env.agent_physical_uuid) == bytes(env.physical_uuid)
    assert bytes(obs.load.digest) == bytes(art.finalizer_identity)
    assert obs.load.byte_len == art.inspection.byte_len
    assert obs.resolution.symbol == b"tiled_gemm_lds_v1"
    assert (obs.resolution.kernarg_segment_bytes, obs.resolution.kernarg_alignment) == (304, 16)
    assert (obs.resources.group_segment_bytes, obs.resources.private_segment_bytes) == (1024, 0)
    completed = loaded.dispatch_and_wait()
    assert any(completed.dispatch_identity)
    receipt = completed.unload()
    assert receipt.executable_object == bytes(obs.load.executable_object)
    rc, ref = oracle.tiled_gemm_arithmetic_v1(16, 16, 16, a, b)
    assert gc.download().view(np.uint32).tolist() == ref.view(np.uint32).tolist()


def test_lifecycle_drop_while_loaded_then_again(gpu, oracle):
    """A loaded lifecycle released without dispatch unloads its module and
    writes nothing; a second lifecycle then loads its own executable (a new
    identity) and computes the product."""
    lc = _lc()
    _, a, b, _ = rv.lds_tile_cases()[0]
    a = np.array(a, np.uint16)
    b = np.array(b, np.uint16)
    ga, gb = gpu.to_device(a), gpu.to_device(b)
    gc = Guarded(gpu, np.full(256, 3.0, np.float32))
    leases = Leases()
    loaded = lc.join_exact_lds_gemm_slice1_v1(ga, gb, gc.body, on_release=leases).load()
    first = bytes(loaded.observation().load.executable_object)
    loaded.release()
    assert leases.drops == 1
    assert gc.unchanged()
    completed = lc.join_exact_lds_gemm_slice1_v1(ga, gb, gc.body).load().dispatch_and_wait()
    assert completed.executable_object != first
    completed.release()  # Drop of a completed lifecycle: terminal unload
    rc, ref = oracle.tiled_gemm_arithmetic_v1(16, 16, 16, a, b)
    assert gc.download().view(np.uint32).tolist() == ref.view(np.uint32).tolist()


def test_lifecycle_context_mismatch_touches_nothing(gpu):
    """A request joined for another device ordinal is refused at load by the
    HIP adapter of device 0, before any load; C is untouched."""
    lc = _lc()
    ga = gpu.to_device(np.zeros(256, np.uint16))
    gb = gpu.to_device(np.zeros(256, np.uint16))
    gc = Guarded(gpu, np.full(256, 5.0, np.float32))
    joined = lc.join_exact_lds_gemm_slice1_v1(ga, gb, gc.body, device=1)
    from fe2o3_amd import _lib
    import ctypes as C
    table = _lib.Fe2o3Slice1AdapterV1()
    assert _lib.lib().fe2o3_lds_gemm_slice1_hip_adapter_v1(0, C.byref(table)) == 0
    h = joined._take()
    err = _lib.Fe2o3Slice1ErrorV1()
    assert _lib.lib().fe2o3_lds_gemm_slice1_load_v1(h.ptr, C.byref(table), C.byref(err)) == -28
    assert lc.KINDS[err.kind] == "ContextIdentity"
    obs = h.observe()
    assert obs.state == lc.FAILED and not obs.holds_executable and not obs.leases_retained
    h.release()
    assert gc.unchanged()
