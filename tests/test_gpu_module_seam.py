"""The runtime seam's module subset (crates/fe2o3-hip-sys/src/lib.rs:144-165:
hipModuleLoad, hipModuleLoadData, hipModuleUnload, hipModuleGetFunction,
hipModuleLaunchKernel) on the GPU, through the C-ABI.

The code object is the library's own slice-1 artifact, which the build
places next to the library (fe2o3_amd/tiled_gemm_lds_v1.co); its SHA-256 is
checked against the lifecycle artifact's finalizer identity, so these are
the bytes the library embeds.  A caller that loads its own code objects
drives it as the reference's typed launch path does: load, resolve the
symbol, launch with the kernel's explicit arguments (three {address,
elements} regions; HIP fills the implicit suffix), synchronize, unload.  The
product is judged on the reference's six-case matrix as in
tests/test_gpu_lifecycle.py: exact cases bit for bit, the others within
64*eps*sum|p| + FLT_MIN.  The kernel writes quiet NaN instead of a product if
the implicit arguments do not describe the launch, so a correct C also
shows HIP initialized them.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os

import numpy as np
import pytest

from golden import reference_vectors as rv
from gpu_util import Guarded

pytestmark = pytest.mark.gpu

FLT_EPS = np.float32(np.finfo(np.float32).eps)
FLT_MIN = np.float32(np.finfo(np.float32).tiny)


class Region(C.Structure):
    _fields_ = [("address", C.c_uint64), ("elements", C.c_uint64)]


def _code_object():
    from fe2o3_amd import _lib, lifecycle
    path = os.path.join(os.path.dirname(_lib.LIB_PATH), "tiled_gemm_lds_v1.co")
    with open(path, "rb") as f:
        data = f.read()
    assert hashlib.sha256(data).digest() == bytes(lifecycle.artifact().finalizer_identity)
    return path, data


def _check(rc, what):
    from fe2o3_amd import _lib
    assert rc == 0, f"{what}: {rc} ({_lib.lib().fe2o3_status_string(rc).decode()})"


def _launch(L, fn, regions, stream):
    params = (C.c_void_p * 3)(*[C.cast(C.pointer(r), C.c_void_p) for r in regions])
    _check(L.fe2o3_rt_module_launch_kernel(fn, 1, 1, 1, 64, 1, 1, 0, stream, params, None),
           "launch")


def _judge(oracle, a, b, got, exact):
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


@pytest.mark.parametrize("from_file", [False, True])
def test_module_seam_six_cases(gpu, oracle, from_file):
    from fe2o3_amd import _lib
    L = _lib.lib()
    path, data = _code_object()
    image = C.create_string_buffer(data, len(data))
    module = C.c_void_p()
    if from_file:
        _check(L.fe2o3_rt_module_load(C.byref(module), path.encode()), "module load")
    else:
        _check(L.fe2o3_rt_module_load_data(C.byref(module), image), "module load data")
    assert module.value
    fn = C.c_void_p()
    _check(L.fe2o3_rt_module_get_function(C.byref(fn), module, b"tiled_gemm_lds_v1"),
           "get function")
    assert fn.value
    stream = gpu.stream()
    try:
        for name, a, b, exact in rv.lds_tile_cases():
            a = np.array(a, np.uint16)
            b = np.array(b, np.uint16)
            ga, gb = Guarded(gpu, a), Guarded(gpu, b)
            gc = Guarded(gpu, np.full(256, np.nan, np.float32))
            regions = [Region(ga.body.ptr, 256), Region(gb.body.ptr, 256),
                       Region(gc.body.ptr, 256)]
            _launch(L, fn, regions, stream.handle)
            _check(L.fe2o3_rt_stream_synchronize(stream.handle), "synchronize")
            assert ga.unchanged() and gb.unchanged() and gc.guards_intact(), name
            _judge(oracle, a, b, gc.download(), exact)
    finally:
        _check(L.fe2o3_rt_module_unload(module), "unload")


def test_module_seam_unknown_symbol_is_an_error(gpu, oracle):
    """A symbol the module does not hold is HIP's error (a positive status)
    and leaves the function handle NULL; the module still unloads.  The
    failed lookup stays in HIP's thread-local last error; the next entry
    point still reports its own launch (0) and computes its product."""
    from fe2o3_amd import _lib
    L = _lib.lib()
    _, data = _code_object()
    image = C.create_string_buffer(data, len(data))
    module = C.c_void_p()
    _check(L.fe2o3_rt_module_load_data(C.byref(module), image), "module load data")
    fn = C.c_void_p(0x1234)
    rc = L.fe2o3_rt_module_get_function(C.byref(fn), module, b"tiled_gemm_lds_v2")
    assert rc > 0 and not fn.value
    _check(L.fe2o3_rt_module_unload(module), "unload")
    m = n = k = 256
    a = oracle.fill_normal_bf16(m * k, 1, 0xA, 1.0 / 16.0)
    b = oracle.fill_normal_bf16(n * k, 1, 0xB, 1.0 / 16.0)
    da, db = gpu.to_device(a), gpu.to_device(b)
    dc = gpu.alloc(m * n, np.uint16)
    rc = L.fe2o3_gemm_bf16_nt(da.ptr, da.count, db.ptr, db.count, dc.ptr, dc.count, m, n, k, None)
    assert rc == 0, rc
    _check(L.fe2o3_rt_device_synchronize(), "synchronize")
    got = oracle.bf16_to_f32(dc.download()).reshape(m, n)
    ref = oracle.gemm_bf16_nt_rows(m, n, k, a, b, 0, m).reshape(m, n)
    assert float(np.max(np.abs(got - ref)) / np.max(np.abs(ref))) <= 1e-2
