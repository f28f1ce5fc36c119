"""Typed kernel launch surface.

Mirrors the reference's generated ``<kernel>_gpu`` modules
(crates/fe2o3-macros/src/lib.rs:1081-1120; the vecadd instance is
crates/fe2o3-host/src/generated_vecadd.rs:37-165):

    k = tiled_gemm_lds_slice1_gpu.Kernel.load(ctx)
    k.prepare(a, b, c).launch(stream)

``load`` checks the device (gfx950 only), ``prepare`` checks every slice's
element type and length against the kernel signature and fails closed with
``Fe2o3Error`` before any launch, and ``launch`` enqueues on the stream and
then synchronizes it, so buffers are quiescent when it returns, as the
reference's typed launch is synchronous by design
(crates/fe2o3-host/src/loaded_kernel.rs:420-432).  The prepared launch holds
its slices, so buffers handed in as temporaries live until it is dropped.
``launch_async`` only enqueues: keep the prepared launch (or the buffers)
until the stream has been synchronized.  The physical argument order is the reference's: one
(pointer, length) pair per slice in declaration order, then the scalars
(examples/tiled_gemm_general_v1/hardware-harness/src/lib.rs:578-597).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .runtime import DeviceBuffer, Fe2o3Error, GpuContext, Stream, check, stream_handle

U16, U32, F32, U8 = np.dtype(np.uint16), np.dtype(np.uint32), np.dtype(np.float32), np.dtype(np.uint8)
ERR_LENGTH = -2


class _Prepared:
    """A checked launch: the flattened arguments, plus the slices themselves,
    held so that a buffer passed as a temporary (``prepare(ctx.to_device(x),
    ...)``) stays allocated until the launch has run; a DeviceBuffer frees
    its memory when it is collected."""

    def __init__(self, kernel: "_TypedKernel", args: tuple, buffers: tuple):
        self.kernel = kernel
        self.args = args
        self.buffers = buffers

    def launch_async(self, stream: Stream | None = None) -> None:
        fn = getattr(_lib.lib(), self.kernel.ENTRY)
        self.kernel.ctx.bind()
        check(fn(*self.args, stream_handle(stream)), self.kernel.ENTRY)

    def launch(self, stream: Stream | None = None) -> None:
        self.launch_async(stream)
        if stream is None:
            self.kernel.ctx.synchronize()
        else:
            stream.synchronize()


class _TypedKernel:
    ENTRY = ""
    # (name, dtype, fixed length or None) per slice, in declaration order
    SLICES: tuple = ()
    # (name, ctypes type) per scalar, in declaration order
    SCALARS: tuple = ()

    def __init__(self, ctx: GpuContext):
        self.ctx = ctx

    @classmethod
    def load(cls, ctx: GpuContext | None = None):
        return cls(ctx or GpuContext.current())

    def prepare(self, *args) -> _Prepared:
        ns, nk = len(self.SLICES), len(self.SCALARS)
        if len(args) != ns + nk:
            raise TypeError(f"{self.ENTRY} takes {ns} slices and {nk} scalars")
        flat = []
        for (name, dtype, fixed), buf in zip(self.SLICES, args[:ns]):
            if buf is None:
                flat += [None, 0]
                continue
            if not isinstance(buf, DeviceBuffer):
                raise TypeError(f"{name} must be a DeviceBuffer")
            if buf.dtype != dtype:
                raise TypeError(f"{name} must hold {dtype}, not {buf.dtype}")
            if fixed is not None and buf.count != fixed:
                raise Fe2o3Error(ERR_LENGTH, f"{self.ENTRY}: {name} length {buf.count} != {fixed}")
            flat += [buf.ptr, buf.count]
        for (name, ctype), value in zip(self.SCALARS, args[ns:]):
            flat.append(ctype(value))
        return _Prepared(self, tuple(flat), tuple(args[:ns]))


def _typed(entry, slices, scalars=()):
    kernel = type("Kernel", (_TypedKernel,), {"ENTRY": entry, "SLICES": tuple(slices),
                                              "SCALARS": tuple(scalars)})
    return type(entry.replace("fe2o3_", "") + "_gpu", (), {"Kernel": kernel})


u32, i32, f32 = C.c_uint32, C.c_int32, C.c_float

# examples/tiled_gemm_v1/src/kernel.rs:63-67
tiled_gemm_lds_slice1_gpu = _typed(
    "fe2o3_tiled_gemm_lds_slice1_v1", [("a", U16, 256), ("b", U16, 256), ("c", F32, 256)])
# examples/tiled_gemm_v1/src/contract.rs:387-427 (the multi-tile plan)
tiled_gemm_v1_gpu = _typed(
    "fe2o3_tiled_gemm_v1", [("a", U16, None), ("b", U16, None), ("c", F32, None)],
    [("m", u32), ("n", u32), ("k", u32)])
# examples/tiled_gemm_general_v1/src/kernel.rs:67-79
tiled_gemm_general_v1_gpu = _typed(
    "fe2o3_tiled_gemm_general_v1", [("a", U16, None), ("b", U16, None), ("c", F32, None)],
    [("m", u32), ("n", u32), ("k", u32), ("lda", u32), ("ldb", u32), ("ldc", u32),
     ("alpha", f32), ("beta", f32)])
# the same kernel under the VectorizedAOnlyBf16GlobalTransferV1 schedule
# (crates/dialect-schedule/src/general_gemm.rs:13-38)
tiled_gemm_general_vector_a_v1_gpu = _typed(
    "fe2o3_tiled_gemm_general_vector_a_v1",
    [("a", U16, None), ("b", U16, None), ("c", F32, None)],
    [("m", u32), ("n", u32), ("k", u32), ("lda", u32), ("ldb", u32), ("ldc", u32),
     ("alpha", f32), ("beta", f32)])
# examples/scalar_gemm_v1/src/kernel.rs:8
scalar_gemm_v1_gpu = _typed(
    "fe2o3_scalar_gemm_v1", [("a", F32, None), ("b", F32, None), ("c", F32, None)],
    [("m", u32), ("n", u32), ("k", u32)])
# scaled-up bf16 NT GEMM (B stored [n, k])
gemm_bf16_nt_gpu = _typed(
    "fe2o3_gemm_bf16_nt", [("a", U16, None), ("b", U16, None), ("c", U16, None)],
    [("m", u32), ("n", u32), ("k", u32)])
# examples/row_softmax_v1/src/kernel.rs:13
row_softmax_v1_gpu = _typed("fe2o3_row_softmax_v1", [("input", F32, 64), ("output", F32, 64)])
row_softmax_gpu = _typed(
    "fe2o3_row_softmax", [("input", F32, None), ("output", F32, None), ("mask", U8, None)],
    [("rows", C.c_uint64), ("cols", C.c_uint64)])
# examples/flash_attention_v1/src/kernel.rs:130-135
flash_attention_causal_f32_b1_h1_n8_d16_v1_gpu = _typed(
    "fe2o3_flash_attention_causal_f32_b1_h1_n8_d16_v1",
    [("q", F32, 128), ("k", F32, 128), ("v", F32, 128), ("output", F32, 128)])
flash_attention_fwd_gpu = _typed(
    "fe2o3_flash_attention_fwd",
    [("q", U16, None), ("k", U16, None), ("v", U16, None), ("o", U16, None), ("lse", F32, None)],
    [("batch", u32), ("heads", u32), ("seq", u32), ("head_dim", u32), ("causal", i32),
     ("scale", f32)])
# examples/moe_top2_v1/src/kernel.rs:102-111
moe_top2_route_f32_t8_e4_k2_c4_v1_gpu = _typed(
    "fe2o3_moe_top2_route_f32_t8_e4_k2_c4_v1",
    [("logits", F32, 32), ("top2_experts", U32, 16), ("requested_counts", U32, 4),
     ("admitted_counts", U32, 4), ("expert_offsets", U32, 5), ("route_slots", U32, 16),
     ("permutation", U32, 16), ("inverse_permutation", U32, 16)])
# examples/moe_expert_v1/src/kernel.rs:30-34, 104-109
moe_expert_gemm_bf16_m16_n16_k16_v1_gpu = _typed(
    "fe2o3_moe_expert_gemm_bf16_m16_n16_k16_v1",
    [("activations", U16, 256), ("weights", U16, 256), ("output", F32, 256)])
moe_expert_combine_f32_t8_k2_o16_v1_gpu = _typed(
    "fe2o3_moe_expert_combine_f32_t8_k2_o16_v1",
    [("compact_output", F32, 256), ("inverse", U32, 16), ("route_weights", F32, 16),
     ("combined_output", F32, 128)])


# ---- functional helpers for the scaled-up paths -------------------------------------

def _call(entry: str, *args, stream: Stream | None = None, sync: bool = True) -> None:
    fn = getattr(_lib.lib(), entry)
    check(fn(*args, stream_handle(stream)), entry)
    if sync:
        if stream is None:
            check(_lib.lib().fe2o3_rt_device_synchronize(), "device synchronize")
        else:
            stream.synchronize()


def _ps(buf: DeviceBuffer | None):
    return (None, 0) if buf is None else (buf.ptr, buf.count)


def moe_top2_route(logits: DeviceBuffer, out: dict, tokens: int, experts: int,
                   capacity: int = 0xFFFFFFFF, stream=None, sync=True) -> None:
    """Top-2 router over bf16 (uint16 buffer) or f32 logits.  ``out`` maps the
    names top2, requested, admitted, offsets, slots, permutation, inverse,
    weights to DeviceBuffers (weights may be absent)."""
    dtype_code = 1 if logits.dtype == U16 else 0
    _call("fe2o3_moe_top2_route", *_ps(logits), dtype_code,
          *_ps(out["top2"]), *_ps(out["requested"]), *_ps(out["admitted"]),
          *_ps(out["offsets"]), *_ps(out["slots"]), *_ps(out["permutation"]),
          *_ps(out["inverse"]), *_ps(out.get("weights")), tokens, experts, capacity,
          stream=stream, sync=sync)


def moe_ffn_workspace_bytes(tokens: int, hidden: int, ffn: int, experts: int) -> int:
    return int(_lib.lib().fe2o3_moe_ffn_workspace_bytes(tokens, hidden, ffn, experts))


def moe_ffn_top2(x, w_gate, w_up, w_down, routing: dict, out, workspace, tokens, hidden, ffn,
                 experts, stream=None, sync=True) -> None:
    _call("fe2o3_moe_ffn_top2", *_ps(x), *_ps(w_gate), *_ps(w_up), *_ps(w_down),
          *_ps(routing["top2"]), *_ps(routing["offsets"]), *_ps(routing["permutation"]),
          *_ps(routing["inverse"]), *_ps(routing["weights"]), *_ps(out),
          workspace.ptr, workspace.nbytes, tokens, hidden, ffn, experts,
          stream=stream, sync=sync)


def moe_ffn_top2_noalloc(x, w_gate, w_up, w_down, routing: dict, out, tokens, hidden, ffn,
                         experts, stream=None, sync=True) -> None:
    """fe2o3_moe_ffn_top2 without a workspace argument: the library's own
    per-device scratch (FE2O3_MOE_NOALLOC_SCRATCH_BYTES), no allocation."""
    _call("fe2o3_moe_ffn_top2_noalloc", *_ps(x), *_ps(w_gate), *_ps(w_up), *_ps(w_down),
          *_ps(routing["top2"]), *_ps(routing["offsets"]), *_ps(routing["permutation"]),
          *_ps(routing["inverse"]), *_ps(routing["weights"]), *_ps(out), tokens, hidden, ffn,
          experts, stream=stream, sync=sync)


def amax_f32(x: DeviceBuffer, amax: DeviceBuffer, stream=None, sync=True) -> None:
    _call("fe2o3_amax_f32", x.ptr, x.count, amax.ptr, stream=stream, sync=sync)


def fp8_scale_from_amax(amax: DeviceBuffer, scale: DeviceBuffer, stream=None, sync=True) -> None:
    _call("fe2o3_fp8_scale_from_amax", amax.ptr, scale.ptr, stream=stream, sync=sync)


def quantize_e4m3(x: DeviceBuffer, scale: DeviceBuffer, q: DeviceBuffer, stream=None,
                  sync=True) -> None:
    _call("fe2o3_quantize_e4m3", x.ptr, x.count, scale.ptr, q.ptr, q.count, stream=stream,
          sync=sync)


# gfx942 FNUZ fp8 formats (FE2O3_FP8_FNUZ_E4M3 / _E5M2)
FNUZ_E4M3, FNUZ_E5M2 = 0, 1


def fp8_fnuz_from_f32(x: DeviceBuffer, q: DeviceBuffer, fmt: int, stream=None,
                      sync=True) -> None:
    """q = Fp8E4M3Fnuz / Fp8E5M2Fnuz::from_f32(x) elementwise
    (crates/fe2o3-device/src/fp8.rs:85-95, 193-203)."""
    _call("fe2o3_fp8_fnuz_from_f32", x.ptr, x.count, q.ptr, q.count, fmt, stream=stream,
          sync=sync)


def fp8_fnuz_to_f32(q: DeviceBuffer, x: DeviceBuffer, fmt: int, stream=None,
                    sync=True) -> None:
    """x = Fp8E4M3Fnuz / Fp8E5M2Fnuz::to_f32(q) elementwise
    (crates/fe2o3-device/src/fp8.rs:92-95, 200-203)."""
    _call("fe2o3_fp8_fnuz_to_f32", q.ptr, q.count, x.ptr, x.count, fmt, stream=stream,
          sync=sync)


def bf16_from_f32(x: DeviceBuffer, out: DeviceBuffer, stream=None, sync=True) -> None:
    """out = Bf16::from_f32(x) elementwise (crates/fe2o3-device/src/half.rs:182-190)."""
    _call("fe2o3_bf16_from_f32", x.ptr, x.count, out.ptr, out.count, stream=stream, sync=sync)


def gemm_fp8_nt(a, b, scale_a, scale_b, c, m, n, k, stream=None, sync=True) -> None:
    _call("fe2o3_gemm_fp8_nt", a.ptr, a.count, b.ptr, b.count, scale_a.ptr, scale_b.ptr,
          c.ptr, c.count, m, n, k, stream=stream, sync=sync)


# examples/wave64_collectives_v1/src/kernel.rs:18-67 (the mask is a scalar
# between the input slice and the three output slices)
def wave64_collectives_v1(input: DeviceBuffer, active_mask: int, reduction: DeviceBuffer,
                          inclusive: DeviceBuffer, exclusive: DeviceBuffer, stream=None,
                          sync=True) -> None:
    _call("fe2o3_wave64_collectives_v1", *_ps(input), C.c_uint64(active_mask & (2**64 - 1)),
          *_ps(reduction), *_ps(inclusive), *_ps(exclusive), stream=stream, sync=sync)


def wave64_collectives_rows(input: DeviceBuffer, masks: DeviceBuffer, reduction: DeviceBuffer,
                            inclusive: DeviceBuffer, exclusive: DeviceBuffer, rows: int,
                            stream=None, sync=True) -> None:
    _call("fe2o3_wave64_collectives_rows", *_ps(input), *_ps(masks), *_ps(reduction),
          *_ps(inclusive), *_ps(exclusive), rows, stream=stream, sync=sync)


# examples/workgroup_sync_v1/src/kernel.rs:18-78
def lds_reduce_i32_v1(values: DeviceBuffer, output: DeviceBuffer, stream=None,
                      sync=True) -> None:
    _call("fe2o3_lds_reduce_i32_v1", *_ps(values), *_ps(output), stream=stream, sync=sync)


# examples/workgroup_sync_v1/src/scoped_atomic.rs:11-32 (target: one u32)
def scoped_atomic_add_u32_v1(values: DeviceBuffer, eligible: DeviceBuffer,
                             target: DeviceBuffer, stream=None, sync=True) -> None:
    _call("fe2o3_scoped_atomic_add_u32_v1", *_ps(values), *_ps(eligible), target.ptr,
          stream=stream, sync=sync)


# crates/fe2o3-host/src/moe_routing_expert_bridge_v1.rs:220-389 on the device;
# record: 4 x u32 {kind, index, expected, actual}
def moe_routing_check(routing: dict, tokens: int, experts: int, capacity: int,
                      record: DeviceBuffer, stream=None, sync=True) -> None:
    _call("fe2o3_moe_routing_check", *_ps(routing["top2"]), *_ps(routing["requested"]),
          *_ps(routing["admitted"]), *_ps(routing["offsets"]), *_ps(routing["slots"]),
          *_ps(routing["permutation"]), *_ps(routing["inverse"]), tokens, experts, capacity,
          *_ps(record), stream=stream, sync=sync)


def kernel_resources(entry: str) -> list[dict]:
    """Every kernel behind C-ABI entry point `entry` with its launch facts and
    the resources the runtime reports for the loaded code object
    (fe2o3_kernel_resources)."""
    L = _lib.lib()
    count = C.c_uint32(0)
    rc = L.fe2o3_kernel_resources(entry.encode(), 0xFFFFFFFF, None, C.byref(count))
    if rc not in (0, -2):
        check(rc, "fe2o3_kernel_resources")
    out = []
    for i in range(count.value):
        rec = _lib.Fe2o3KernelResources()
        check(L.fe2o3_kernel_resources(entry.encode(), i, C.byref(rec), C.byref(count)),
              "fe2o3_kernel_resources")
        out.append({name: (getattr(rec, name).decode() if name == "kernel" else getattr(rec, name))
                    for name, _ in rec._fields_})
    return out


def fill_normal_bf16(buf: DeviceBuffer, seed: int, domain: int, scale: float, first: int = 0,
                     stream=None, sync=True) -> None:
    _call("fe2o3_fill_normal_bf16", buf.ptr, buf.count, seed, domain, scale, first,
          stream=stream, sync=sync)


def fill_normal_f32(buf: DeviceBuffer, seed: int, domain: int, scale: float, first: int = 0,
                    stream=None, sync=True) -> None:
    _call("fe2o3_fill_normal_f32", buf.ptr, buf.count, seed, domain, scale, first,
          stream=stream, sync=sync)


def fill_uniform_f32(buf: DeviceBuffer, seed: int, domain: int, first: int = 0, stream=None,
                     sync=True) -> None:
    _call("fe2o3_fill_uniform_f32", buf.ptr, buf.count, seed, domain, first, stream=stream,
          sync=sync)
