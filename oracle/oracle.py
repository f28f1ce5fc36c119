"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, always as the checker.  The product package
(fe2o3_amd) never imports this module.

Every function here is a thin numpy wrapper over the C restatement of the
reference oracles; the C sources cite the reference file:line they follow.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")

OK = 0
ERR_LENGTH = -2
ERR_SHAPE = -3
ERR_STRIDE = -4
ERR_NONFINITE = -5
ERR_SUBNORMAL = -6
ERR_ALPHABET = -7
ERR_INTERMEDIATE = -8
ERR_MISMATCH = -9
ERR_POLICY = -10
ERR_EMPTY = -11
ERR_TOO_LARGE = -12
ERR_NO_ACTIVE = -13
ERR_WEIGHTS = -14
ERR_ROUTING = -15
ERR_OVERFLOW = -16
ERR_SUM = -17
ERR_INFINITE = -18
DROP_ROUTE = 0xFFFFFFFF


def build() -> str:
    """Compile liboracle.so from the C sources with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    i32, u32, u64, f32 = C.c_int32, C.c_uint32, C.c_uint64, C.c_float
    vp = C.c_void_p
    sig = {
        "fe2o3o_bf16_from_f32": (C.c_uint16, [f32]),
        "fe2o3o_bf16_to_f32": (f32, [C.c_uint16]),
        "fe2o3o_bf16_from_f32_array": (None, [f32p, u16p, C.c_size_t]),
        "fe2o3o_bf16_to_f32_array": (None, [u16p, f32p, C.c_size_t]),
        "fe2o3o_mix64": (u64, [u64]),
        "fe2o3o_generate_inputs_v1": (None, [u32, u32, u32, u64, vp, vp]),
        "fe2o3o_validate_evidence_inputs_v1": (
            i32, [u32, u32, u32, vp, u64, vp, u64, C.POINTER(i32), C.POINTER(u64)]),
        "fe2o3o_counter_normal": (f32, [u64, u64, u64]),
        "fe2o3o_counter_uniform_pm1": (f32, [u64, u64, u64]),
        "fe2o3o_fill_normal_bf16": (None, [u16p, u64, u64, u64, f32, u64]),
        "fe2o3o_fill_normal_f32": (None, [f32p, u64, u64, u64, f32, u64]),
        "fe2o3o_fill_uniform_f32": (None, [f32p, u64, u64, u64, u64]),
        "fe2o3o_tiled_gemm_arithmetic_v1": (i32, [u32, u32, u32, vp, u64, vp, u64, vp]),
        "fe2o3o_gemm_spec_checked": (
            i32, [u64, u64, u64, u64, u64, u64, C.POINTER(u64), C.POINTER(u64), C.POINTER(u64)]),
        "fe2o3o_evaluate_source": (
            i32, [u64, u64, u64, u64, u64, u64, vp, u64, vp, u64, vp, u64, f32, f32, vp]),
        "fe2o3o_build_hardware_expectation": (
            i32, [u64, u64, u64, u64, u64, u64, vp, u64, vp, u64, vp, u64, f32, f32, vp]),
        "fe2o3o_compare_hardware": (
            i32, [f32p, f32p, u64, i32, f32, f32, u32, f32p, C.POINTER(u32), C.POINTER(u64)]),
        "fe2o3o_ulp_distance": (u32, [f32, f32]),
        "fe2o3o_general_reference_v1": (
            i32, [u32, u32, u32, u32, u32, u32, vp, u64, vp, u64, vp, u64, f32, f32, vp, u64p]),
        "fe2o3o_row_major_xor4": (i32, [u32, u32, C.POINTER(u32)]),
        "fe2o3o_scalar_gemm": (None, [u32, u32, u32, vp, vp, vp]),
        "fe2o3o_scalar_gemm_inputs": (None, [u64, u64, vp, vp]),
        "fe2o3o_gemm_bf16_nt_rows": (None, [u32, u32, u32, u16p, u16p, u32, u32, f32p, i32]),
        "fe2o3o_gemm_bf16_nt_points": (None, [u32, u16p, u16p, u64, f32p, i32]),
        "fe2o3o_gemm_f32_rows": (None, [u32, u32, u32, f32p, f32p, u32, u32, f32p, i32]),
        "fe2o3o_flash_attention_v1": (i32, [vp, u64, vp, u64, vp, u64, vp, u64, vp, vp]),
        "fe2o3o_flash_attention_rows_bf16": (
            i32, [u16p, u16p, u16p, u32, u32, i32, f32, u32p, u32p, u64, f32p, f32p, i32]),
        "fe2o3o_row_softmax_oracle_v1": (i32, [vp, u64, vp, vp, vp]),
        "fe2o3o_compare_row_softmax_v1": (
            i32, [f32p, f32p, u64, vp, f32, f32, f32, u32, C.POINTER(u64)]),
        "fe2o3o_row_softmax_reference_v1": (i32, [f32p, f32p]),
        "fe2o3o_row_softmax_rows": (i32, [f32p, u64, u64, f32p, i32]),
        "fe2o3o_row_softmax_check_rows": (
            i32, [f32p, f32p, u64, u64, f32, f32, f32, u32, i32, C.POINTER(C.c_double)]),
        "fe2o3o_moe_top2_route": (
            i32, [vp, u32, u32, u32, vp, vp, vp, vp, vp, vp, vp]),
        "fe2o3o_moe_select_top2_running": (None, [f32p, u32, u32p]),
        "fe2o3o_moe_top2_weights": (None, [f32p, u32, u32, u32p, f32p]),
        "fe2o3o_moe_expert_independent_v1": (
            i32, [vp, vp, u64, vp, u64, vp, u64, vp, vp, vp, vp, vp, vp, vp]),
        "fe2o3o_moe_expert_pipeline_v1": (
            i32, [vp, vp, u64, vp, u64, vp, u64, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
        "fe2o3o_moe_ffn_route": (None, [u16p, u16p, u16p, u16p, u32, u32, u16p, f32p]),
        "fe2o3o_moe_ffn_routes": (None, [u16p, u16p, u16p, u16p, u32, u32, u32p, u32p, u64, f32p,
                                         i32]),
        "fe2o3o_fp8e4m3_from_f32": (C.c_uint8, [f32]),
        "fe2o3o_fp8e4m3_to_f32": (f32, [C.c_uint8]),
        "fe2o3o_fnuz_from_f32_bits": (C.c_uint8, [u32, i32]),
        "fe2o3o_fnuz_to_f32_bits": (u32, [C.c_uint8, i32]),
        "fe2o3o_fnuz_from_f32_array": (None, [f32p, u64, i32, u8p]),
        "fe2o3o_amax_f32": (f32, [f32p, u64, i32]),
        "fe2o3o_quantize_e4m3": (None, [f32p, u64, f32, u8p, i32]),
        "fe2o3o_gemm_fp8_points": (None, [u32, u8p, u8p, u64, f32, f32p, u16p, i32]),
        "fe2o3o_gemm_fp8_nt_rows": (None, [u32, u32, u8p, u8p, f32, u32, u32, f32p, i32]),
        "fe2o3o_wave64_collectives_compute": (None, [f32p, u64, f32p, f32p, f32p]),
        "fe2o3o_wave64_collectives_v1": (i32, [f32p, u64, f32p, f32p, f32p]),
        "fe2o3o_lds_reduce_i32_v1": (i32, [vp, vp]),
        "fe2o3o_atomic_add_u32_v1": (i32, [u32, u32p, u32p, u32p]),
        "fe2o3o_moe_routing_check": (
            i32, [u32p, u32p, u32p, u32p, u32p, u32p, u32p, u32, u32, u32, u32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _ptr(a):
    """Pointer of a numpy array, or None for empty/None (the C side never
    dereferences a zero-length operand)."""
    if a is None:
        return None
    return a.ctypes.data if a.size else None


def _threads() -> int:
    """Default OpenMP width: the CPUs this process may run on (its affinity
    set; os.cpu_count() can report far more cores than a container grants),
    capped by OMP_NUM_THREADS when that is set (a GPU box sets it to the CPU
    share of its GPU)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- numeric vocabulary -----------------------------------------------------

def bf16_from_f32(x) -> np.ndarray:
    x = _c(np.atleast_1d(x), np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().fe2o3o_bf16_from_f32_array(x.ravel(), out.ravel(), x.size)
    return out


def bf16_to_f32(b) -> np.ndarray:
    b = _c(np.atleast_1d(b), np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def mix64(v: int) -> int:
    return lib().fe2o3o_mix64(v)


# ---- generators -------------------------------------------------------------

def generate_inputs_v1(m, n, k, seed):
    empty = m == 0 or n == 0
    a = np.zeros(0 if empty else m * k, np.uint16)
    b = np.zeros(0 if empty else k * n, np.uint16)
    lib().fe2o3o_generate_inputs_v1(m, n, k, seed, _ptr(a), _ptr(b))
    return a, b


def validate_evidence_inputs_v1(m, n, k, a, b):
    a = _c(a, np.uint16)
    b = _c(b, np.uint16)
    op = C.c_int32(-1)
    idx = C.c_uint64(0)
    rc = lib().fe2o3o_validate_evidence_inputs_v1(
        m, n, k, _ptr(a), a.size, _ptr(b), b.size, C.byref(op), C.byref(idx))
    return rc, op.value, idx.value


def fill_normal_bf16(n, seed, domain, scale, first=0):
    out = np.empty(n, np.uint16)
    lib().fe2o3o_fill_normal_bf16(out, n, seed, domain, scale, first)
    return out


def fill_normal_f32(n, seed, domain, scale, first=0):
    out = np.empty(n, np.float32)
    lib().fe2o3o_fill_normal_f32(out, n, seed, domain, scale, first)
    return out


def fill_uniform_f32(n, seed, domain, first=0):
    out = np.empty(n, np.float32)
    lib().fe2o3o_fill_uniform_f32(out, n, seed, domain, first)
    return out


# ---- GEMM ---------------------------------------------------------------------

def tiled_gemm_arithmetic_v1(m, n, k, a, b):
    a = _c(a, np.uint16)
    b = _c(b, np.uint16)
    out = np.zeros(m * n, np.float32)
    rc = lib().fe2o3o_tiled_gemm_arithmetic_v1(m, n, k, _ptr(a), a.size, _ptr(b), b.size, _ptr(out))
    return rc, out


def gemm_spec_checked(m, n, k, lda, ldb, ldc):
    la, lb, lc = C.c_uint64(), C.c_uint64(), C.c_uint64()
    rc = lib().fe2o3o_gemm_spec_checked(m, n, k, lda, ldb, ldc, C.byref(la), C.byref(lb), C.byref(lc))
    return rc, (la.value, lb.value, lc.value)


def evaluate_source(m, n, k, lda, ldb, ldc, a, b, c, alpha, beta):
    a, b, c = _c(a, np.uint16), _c(b, np.uint16), _c(c, np.float32)
    out = np.zeros(m * n, np.float32)
    rc = lib().fe2o3o_evaluate_source(m, n, k, lda, ldb, ldc, _ptr(a), a.size, _ptr(b), b.size,
                                      _ptr(c), c.size, alpha, beta, _ptr(out))
    return rc, out


def build_hardware_expectation(m, n, k, lda, ldb, ldc, a, b, c, alpha, beta):
    a, b, c = _c(a, np.uint16), _c(b, np.uint16), _c(c, np.float32)
    out = np.zeros(m * n, np.float32)
    rc = lib().fe2o3o_build_hardware_expectation(
        m, n, k, lda, ldb, ldc, _ptr(a), a.size, _ptr(b), b.size, _ptr(c), c.size, alpha, beta,
        _ptr(out))
    return rc, out


EXACT_BITS = 0
BOUNDED = 1


def compare_hardware(expected, observed, policy=EXACT_BITS, max_abs=0.0, max_rel=0.0, max_ulps=0):
    e = _c(expected, np.float32).ravel()
    o = _c(observed, np.float32).ravel()
    rep = np.zeros(2, np.float32)
    ulp = C.c_uint32(0)
    bad = C.c_uint64(0)
    rc = lib().fe2o3o_compare_hardware(e, o, e.size, policy, max_abs, max_rel, max_ulps, rep,
                                       C.byref(ulp), C.byref(bad))
    return rc, {"max_abs": float(rep[0]), "max_rel": float(rep[1]), "max_ulp": ulp.value,
                "bad_index": bad.value}


def ulp_distance(x, y):
    return lib().fe2o3o_ulp_distance(x, y)


def general_reference_v1(m, n, k, lda, ldb, ldc, a, b, c, alpha, beta):
    a, b, c = _c(a, np.uint16), _c(b, np.uint16), _c(c, np.float32)
    out = np.zeros(m * n, np.float32)
    trace = np.zeros(8, np.uint64)
    rc = lib().fe2o3o_general_reference_v1(m, n, k, lda, ldb, ldc, _ptr(a), a.size, _ptr(b),
                                           b.size, _ptr(c), c.size, alpha, beta, _ptr(out), trace)
    names = ["workgroups", "reduction_phases", "publish_barriers", "reuse_barriers",
             "a_zero_fills", "b_zero_fills", "output_stores", "c_predicated_stores"]
    return rc, out, dict(zip(names, (int(t) for t in trace)))


def row_major_xor4(row, col):
    p = C.c_uint32()
    rc = lib().fe2o3o_row_major_xor4(row, col, C.byref(p))
    return rc, p.value


def scalar_gemm(m, n, k, a, b):
    a, b = _c(a, np.float32), _c(b, np.float32)
    out = np.zeros(m * n, np.float32)
    lib().fe2o3o_scalar_gemm(m, n, k, _ptr(a), _ptr(b), _ptr(out))
    return out


def scalar_gemm_inputs(a_len, b_len):
    a = np.zeros(a_len, np.float32)
    b = np.zeros(b_len, np.float32)
    lib().fe2o3o_scalar_gemm_inputs(a_len, b_len, _ptr(a), _ptr(b))
    return a, b


def gemm_bf16_nt_rows(m, n, k, a, b, row_begin, row_end, threads=0):
    out = np.zeros((row_end - row_begin) * n, np.float32)
    lib().fe2o3o_gemm_bf16_nt_rows(m, n, k, _c(a, np.uint16).ravel(), _c(b, np.uint16).ravel(),
                                   row_begin, row_end, out, threads or _threads())
    return out


def gemm_bf16_nt_points(k, a_rows, b_cols, threads=0):
    a_rows = _c(a_rows, np.uint16)
    b_cols = _c(b_cols, np.uint16)
    pts = a_rows.shape[0]
    out = np.zeros(pts, np.float32)
    lib().fe2o3o_gemm_bf16_nt_points(k, a_rows.ravel(), b_cols.ravel(), pts, out,
                                     threads or _threads())
    return out


def gemm_f32_rows(m, n, k, a, b, row_begin, row_end, threads=0):
    out = np.zeros((row_end - row_begin) * n, np.float32)
    lib().fe2o3o_gemm_f32_rows(m, n, k, _c(a, np.float32).ravel(), _c(b, np.float32).ravel(),
                               row_begin, row_end, out, threads or _threads())
    return out


# ---- attention / softmax ------------------------------------------------------

def flash_attention_v1(q, k, v, out_len=128):
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    out = np.full(out_len, np.nan, np.float32)
    mx = np.zeros(8, np.float64)
    den = np.zeros(8, np.float64)
    rc = lib().fe2o3o_flash_attention_v1(_ptr(q), q.size, _ptr(k), k.size, _ptr(v), v.size,
                                         _ptr(out), out.size, _ptr(mx), _ptr(den))
    return rc, out, mx, den


def flash_attention_rows_bf16(q, k, v, s, d, causal, scale, bh, rows, threads=0):
    bh = _c(bh, np.uint32)
    rows = _c(rows, np.uint32)
    out = np.zeros(rows.size * d, np.float32)
    lse = np.zeros(rows.size, np.float32)
    rc = lib().fe2o3o_flash_attention_rows_bf16(
        _c(q, np.uint16).ravel(), _c(k, np.uint16).ravel(), _c(v, np.uint16).ravel(), s, d,
        int(causal), scale, bh, rows, rows.size, out, lse, threads or _threads())
    return rc, out.reshape(rows.size, d), lse


def row_softmax_oracle_v1(x, mask=None, out=None):
    x = _c(x, np.float32)
    if out is None:
        out = np.full(x.size, np.nan, np.float32)
    m = None if mask is None else _c(mask, np.uint8)
    state = np.zeros(3, np.float64)
    rc = lib().fe2o3o_row_softmax_oracle_v1(_ptr(x), x.size, _ptr(m), out.ctypes.data, _ptr(state))
    return rc, out, {"maximum": state[0], "denominator": state[1], "active": int(state[2])}


GFX_SOFTMAX_POLICY = dict(abs_tol=3.0e-6, rel_tol=3.0e-5, sum_tol=6.0e-5, max_ulps=64)


def compare_row_softmax_v1(expected, actual, mask=None, abs_tol=3.0e-6, rel_tol=3.0e-5,
                           sum_tol=6.0e-5, max_ulps=64):
    e, a = _c(expected, np.float32), _c(actual, np.float32)
    m = None if mask is None else _c(mask, np.uint8)
    bad = C.c_uint64(0)
    rc = lib().fe2o3o_compare_row_softmax_v1(e, a, e.size, _ptr(m), abs_tol, rel_tol, sum_tol,
                                             max_ulps, C.byref(bad))
    return rc, bad.value


def row_softmax_reference_v1(x):
    x = _c(x, np.float32)
    out = np.zeros(64, np.float32)
    rc = lib().fe2o3o_row_softmax_reference_v1(x, out)
    return rc, out


def row_softmax_check_rows(x, y, rows, cols, threads=0, abs_tol=3.0e-6, rel_tol=3.0e-5,
                           sum_tol=6.0e-5, max_ulps=64):
    """Every row of y against the f64 oracle of the same row of x under the
    comparison policy (default: GFX_SOFTMAX_POLICY), in C over OpenMP.
    Returns (rc, stats): failing rows, the first failing row (rows if none),
    max abs difference, max |oracle|, max |f64 row sum - 1|."""
    x = _c(x, np.float32).ravel()
    y = _c(y, np.float32).ravel()
    assert x.size == y.size == rows * cols
    st = (C.c_double * 5)()
    rc = lib().fe2o3o_row_softmax_check_rows(x, y, rows, cols, abs_tol, rel_tol, sum_tol,
                                             max_ulps, threads or _threads(), st)
    return rc, {"failing_rows": int(st[0]), "first_failing_row": int(st[1]),
                "max_abs_diff": st[2], "max_ref": st[3], "max_row_sum_err": st[4]}


def row_softmax_rows(x, rows, cols, threads=0):
    x = _c(x, np.float32).ravel()
    out = np.zeros(rows * cols, np.float32)
    rc = lib().fe2o3o_row_softmax_rows(x, rows, cols, out, threads or _threads())
    return rc, out.reshape(rows, cols)


# ---- MoE ------------------------------------------------------------------------

def moe_top2_route(logits, tokens, experts, capacity=DROP_ROUTE, fill=0xABABABAB):
    lg = _c(logits, np.float32).ravel()
    r = 2 * tokens
    outs = {
        "top2_experts": np.full(r, fill, np.uint32),
        "requested_counts": np.full(experts, fill, np.uint32),
        "admitted_counts": np.full(experts, fill, np.uint32),
        "expert_offsets": np.full(experts + 1, fill, np.uint32),
        "route_slots": np.full(r, fill, np.uint32),
        "permutation": np.full(r, fill, np.uint32),
        "inverse": np.full(r, fill, np.uint32),
    }
    rc = lib().fe2o3o_moe_top2_route(
        _ptr(lg), tokens, experts, capacity,
        *(outs[k].ctypes.data for k in ("top2_experts", "requested_counts", "admitted_counts",
                                        "expert_offsets", "route_slots", "permutation",
                                        "inverse")))
    return rc, outs


def moe_select_top2_running(row):
    row = _c(row, np.float32)
    out = np.zeros(2, np.uint32)
    lib().fe2o3o_moe_select_top2_running(row, row.size, out)
    return out


def moe_top2_weights(logits, tokens, experts, top2):
    w = np.zeros(2 * tokens, np.float32)
    lib().fe2o3o_moe_top2_weights(_c(logits, np.float32).ravel(), tokens, experts,
                                  _c(top2, np.uint32), w)
    return w


def moe_expert_independent_v1(logits, acts, weights, route_weights, routing):
    acts, weights = _c(acts, np.uint16), _c(weights, np.uint16)
    rw = _c(route_weights, np.float32)
    tiles = np.zeros(4 * 256, np.float32)
    compact = np.zeros(16 * 16, np.float32)
    combined = np.zeros(8 * 16, np.float32)
    route_out = np.zeros(16 * 16, np.float32)
    rc = lib().fe2o3o_moe_expert_independent_v1(
        _c(logits, np.float32).ctypes.data, _ptr(acts), acts.size, _ptr(weights), weights.size,
        _ptr(rw), rw.size, routing["top2_experts"].ctypes.data,
        routing["expert_offsets"].ctypes.data, routing["inverse"].ctypes.data,
        tiles.ctypes.data, compact.ctypes.data, combined.ctypes.data, route_out.ctypes.data)
    return rc, {"expert_output_tiles": tiles, "compact_output": compact,
                "combined_output": combined, "route_output": route_out}


def moe_expert_pipeline_v1(logits, acts, weights, route_weights, routing):
    acts, weights = _c(acts, np.uint16), _c(weights, np.uint16)
    rw = _c(route_weights, np.float32)
    at = np.zeros(4 * 256, np.uint16)
    tiles = np.zeros(4 * 256, np.float32)
    compact = np.zeros(16 * 16, np.float32)
    combined = np.zeros(8 * 16, np.float32)
    rc = lib().fe2o3o_moe_expert_pipeline_v1(
        _c(logits, np.float32).ctypes.data, _ptr(acts), acts.size, _ptr(weights), weights.size,
        _ptr(rw), rw.size, routing["top2_experts"].ctypes.data,
        routing["admitted_counts"].ctypes.data, routing["expert_offsets"].ctypes.data,
        routing["permutation"].ctypes.data, routing["inverse"].ctypes.data, at.ctypes.data,
        tiles.ctypes.data, compact.ctypes.data, combined.ctypes.data)
    return rc, {"activation_tiles": at, "expert_output_tiles": tiles, "compact_output": compact,
                "combined_output": combined}


def moe_ffn_route(x, w_gate, w_up, w_down, h, f):
    hidden = np.zeros(f, np.uint16)
    y = np.zeros(h, np.float32)
    lib().fe2o3o_moe_ffn_route(_c(x, np.uint16), _c(w_gate, np.uint16).ravel(),
                               _c(w_up, np.uint16).ravel(), _c(w_down, np.uint16).ravel(), h, f,
                               hidden, y)
    return hidden, y


def moe_ffn_routes(x, w_gate, w_up, w_down, h, f, tokens, experts, threads=0):
    """Expert outputs y [n, h] (f32) of the (token, expert) pairs; x is
    [tokens, h] bf16 bits, weights [E, F, H] / [E, H, F]."""
    tok, exp = _c(tokens, np.uint32).ravel(), _c(experts, np.uint32).ravel()
    y = np.zeros((tok.size, h), np.float32)
    lib().fe2o3o_moe_ffn_routes(_c(x, np.uint16).ravel(), _c(w_gate, np.uint16).ravel(),
                                _c(w_up, np.uint16).ravel(), _c(w_down, np.uint16).ravel(), h, f,
                                tok, exp, tok.size, y.ravel(), threads or _threads())
    return y


# ---- fp8 -------------------------------------------------------------------------

def fp8_from_f32(x: float) -> int:
    return lib().fe2o3o_fp8e4m3_from_f32(x)


def fp8_to_f32(b: int) -> float:
    return lib().fe2o3o_fp8e4m3_to_f32(b)


# gfx942 FNUZ fp8: format 0 = E4M3 FNUZ, 1 = E5M2 FNUZ
FNUZ_E4M3, FNUZ_E5M2 = 0, 1


def fnuz_from_f32_bits(bits: int, fmt: int) -> int:
    return lib().fe2o3o_fnuz_from_f32_bits(bits, fmt)


def fnuz_to_f32_bits(q: int, fmt: int) -> int:
    return lib().fe2o3o_fnuz_to_f32_bits(q, fmt)


def fnuz_from_f32(x, fmt: int) -> np.ndarray:
    x = _c(x, np.float32).ravel()
    out = np.zeros(x.size, np.uint8)
    lib().fe2o3o_fnuz_from_f32_array(x, x.size, fmt, out)
    return out


def fnuz_decode_table(fmt: int) -> np.ndarray:
    """f32 bit patterns of the 256 codes"""
    return np.array([fnuz_to_f32_bits(i, fmt) for i in range(256)], np.uint32)


def fp8_decode_table() -> np.ndarray:
    return np.array([fp8_to_f32(i) for i in range(256)], np.float32)


def amax_f32(x, threads=0):
    x = _c(x, np.float32).ravel()
    return lib().fe2o3o_amax_f32(x, x.size, threads or _threads())


def quantize_e4m3(x, scale, threads=0):
    x = _c(x, np.float32).ravel()
    out = np.zeros(x.size, np.uint8)
    lib().fe2o3o_quantize_e4m3(x, x.size, scale, out, threads or _threads())
    return out


def gemm_fp8_points(k, a_rows, b_cols, scale_ab, threads=0):
    a_rows, b_cols = _c(a_rows, np.uint8), _c(b_cols, np.uint8)
    p = a_rows.shape[0]
    of = np.zeros(p, np.float32)
    ob = np.zeros(p, np.uint16)
    lib().fe2o3o_gemm_fp8_points(k, a_rows.ravel(), b_cols.ravel(), p, scale_ab, of, ob,
                                 threads or _threads())
    return of, ob


def gemm_fp8_nt_rows(n, k, a, b, scale_ab, row_begin, row_end, threads=0):
    """f32 values (before bf16 narrowing) of output rows row_begin..row_end-1
    of (sa*sb) * A_q B_q^T; a is [m, k], b [n, k] e4m3 bytes."""
    out = np.zeros((row_end - row_begin) * n, np.float32)
    lib().fe2o3o_gemm_fp8_nt_rows(n, k, _c(a, np.uint8).ravel(), _c(b, np.uint8).ravel(),
                                  scale_ab, row_begin, row_end, out, threads or _threads())
    return out.reshape(row_end - row_begin, n)


# ---- collectives, workgroup sync, routing consistency (sync.c) ----------------------------

ROUTING_CHECK_KINDS = (
    "ok", "expert_out_of_range", "duplicate_token_expert", "requested_count", "capacity",
    "admitted_count", "first_offset", "nonmonotone_offsets", "offset_mismatch",
    "plan_offset_order", "plan_capacity", "slot_out_of_range", "duplicate_slot", "stable_slot",
    "inverse", "permutation", "prefix_hole", "permutation_route", "permutation_tail")


def wave64_collectives(x, mask, admit=True):
    """(rc, reduction, inclusive, exclusive) for 64 f32 inputs.  admit=True
    applies the reference's exact-corpus admission (finite integers in
    [-1024, 1024]); admit=False computes the fixed-order rounds for any
    input.  Outputs are NaN-filled when rejected."""
    x = _c(x, np.float32)
    outs = [np.full(64, np.nan, np.float32) for _ in range(3)]
    if admit:
        rc = lib().fe2o3o_wave64_collectives_v1(x, int(mask) & 0xFFFFFFFFFFFFFFFF, *outs)
    else:
        lib().fe2o3o_wave64_collectives_compute(x, int(mask) & 0xFFFFFFFFFFFFFFFF, *outs)
        rc = OK
    return rc, outs[0], outs[1], outs[2]


def lds_reduce_i32(values):
    v = _c(values, np.int32)
    out = np.zeros(1, np.int32)
    rc = lib().fe2o3o_lds_reduce_i32_v1(v.ctypes.data, out.ctypes.data)
    return rc, int(out[0])


def atomic_add_u32(initial, values, eligible):
    out = np.zeros(1, np.uint32)
    rc = lib().fe2o3o_atomic_add_u32_v1(initial, _c(values, np.uint32),
                                        _c(eligible, np.uint32), out)
    return rc, int(out[0])


def moe_routing_check(outs, tokens, experts, capacity=DROP_ROUTE):
    """First inconsistency of a routing output (dict as moe_top2_route
    returns) as (kind name, index, expected, actual)."""
    rec = np.zeros(4, np.uint32)
    rc = lib().fe2o3o_moe_routing_check(
        *(_c(outs[k], np.uint32) for k in ("top2_experts", "requested_counts", "admitted_counts",
                                           "expert_offsets", "route_slots", "permutation",
                                           "inverse")),
        tokens, experts, capacity, rec)
    assert rc == OK
    return ROUTING_CHECK_KINDS[rec[0]], int(rec[1]), int(rec[2]), int(rec[3])
