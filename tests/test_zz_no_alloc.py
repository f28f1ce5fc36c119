"""The allocation-free MoE FFN entry point (fe2o3_moe_ffn_top2_noalloc),
through the C-ABI, against fe2o3_moe_ffn_top2 with a caller workspace: bit
for bit on two calls in a row, the second with fewer tokens (the scratch
keeps the first call's contents), at a small shape and at the BASELINE
layer's hidden 4096 / ffn 14336 with serving-size token counts; sizes above
the scratch are rejected before any launch."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import Guarded

pytestmark = pytest.mark.gpu


def _k():
    from fe2o3_amd import kernels
    return kernels


def _routed(gpu, tokens, experts, seed):
    kern = _k()
    lg = gpu.alloc(tokens * experts, np.uint16)
    kern.fill_normal_bf16(lg, seed, 0x10617, 1.0)
    n = 2 * tokens
    r = {"top2": gpu.alloc(n, np.uint32), "requested": gpu.alloc(experts, np.uint32),
         "admitted": gpu.alloc(experts, np.uint32), "offsets": gpu.alloc(experts + 1, np.uint32),
         "slots": gpu.alloc(n, np.uint32), "permutation": gpu.alloc(n, np.uint32),
         "inverse": gpu.alloc(n, np.uint32), "weights": gpu.alloc(n, np.float32)}
    kern.moe_top2_route(lg, r, tokens, experts)
    return r


@pytest.mark.parametrize("hidden,ffn,experts,calls", [
    (512, 1024, 8, (300, 100)),
    (4096, 14336, 8, (256, 64)),
])
def test_noalloc_matches_workspace_entry(gpu, hidden, ffn, experts, calls):
    kern = _k()
    wsz = experts * ffn * hidden
    w = [gpu.alloc(wsz, np.uint16) for _ in range(3)]
    for i, dom in enumerate((0x6A7E, 0x0B0B, 0xD0D0)):
        kern.fill_normal_bf16(w[i], 5, dom, 0.02)
    for call, tokens in enumerate(calls):
        x = gpu.alloc(tokens * hidden, np.uint16)
        kern.fill_normal_bf16(x, 11 + call, 0xAC7, 1.0)
        r = _routed(gpu, tokens, experts, 11 + call)
        ws = gpu.alloc(kern.moe_ffn_workspace_bytes(tokens, hidden, ffn, experts), np.uint8)
        want = Guarded(gpu, np.full(tokens * hidden, 0x7FDE, np.uint16))
        kern.moe_ffn_top2(x, w[0], w[1], w[2], r, want.body, ws, tokens, hidden, ffn, experts)
        got = Guarded(gpu, np.full(tokens * hidden, 0x7FDE, np.uint16))
        kern.moe_ffn_top2_noalloc(x, w[0], w[1], w[2], r, got.body, tokens, hidden, ffn, experts)
        assert got.guards_intact() and want.guards_intact()
        g, h = got.download(), want.download()
        assert np.any(h != 0)
        assert g.tobytes() == h.tobytes(), (call, tokens, int(np.sum(g != h)))


def test_noalloc_rejects_sizes_above_its_scratch(gpu):
    from fe2o3_amd import _lib
    L = _lib.lib()
    limit = 64 << 20
    assert L.fe2o3_moe_ffn_workspace_bytes(481, 4096, 14336, 8) <= limit
    assert L.fe2o3_moe_ffn_workspace_bytes(482, 4096, 14336, 8) > limit
    out = Guarded(gpu, np.full(16, 0x7FDE, np.uint16))
    rc = L.fe2o3_moe_ffn_top2_noalloc(None, 0, None, 0, None, 0, None, 0, None, 0, None, 0,
                                      None, 0, None, 0, None, 0, out.body.ptr, 16, 482, 4096,
                                      14336, 8, None)
    assert rc == -22
    assert out.unchanged()
