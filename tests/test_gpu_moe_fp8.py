"""GPU parity tests for the top-2 MoE path and the fp8 quantized GEMM path,
through the C-ABI, against the CPU oracle restatements.

Routing (indices, counts, offsets, slots, permutation, inverse) is integer
work and must be bit-exact; gating weights within 1e-6 relative with pairs
summing to exactly 1; the expert FFN and fp8 GEMM outputs within rel-err
1e-2 (bf16 outputs); fp8 encoding bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from golden import reference_vectors as rv
from gpu_util import GUARD, Guarded, assert_same, bf16_to_f32, rel_err

pytestmark = pytest.mark.gpu

ROUTE_KEYS = ["top2_experts", "requested_counts", "admitted_counts", "expert_offsets",
              "route_slots", "permutation", "inverse"]


def _k():
    from fe2o3_amd import kernels
    return kernels


# ---- router: exact profile -------------------------------------------------------------

@pytest.mark.parametrize("name", list(rv.MOE_VECTORS))
def test_route_profile_bit_exact(gpu, oracle, name):
    """examples/moe_top2_v1/src/vectors.rs:14-117 through the fixed
    T8/E4/K2/C4 entry point; every output array bit-equal to the oracle."""
    logits = np.array(rv.MOE_VECTORS[name], np.float32)
    rc, ref = oracle.moe_top2_route(logits, 8, 4, 4)
    assert rc == 0
    lens = [16, 4, 4, 5, 16, 16, 16]
    outs = [Guarded(gpu, np.full(n, 0xABABABAB, np.uint32)) for n in lens]
    gl = Guarded(gpu, logits)
    _k().moe_top2_route_f32_t8_e4_k2_c4_v1_gpu.Kernel.load(gpu).prepare(
        gl.body, *[o.body for o in outs]).launch()
    assert gl.unchanged()
    for key, o in zip(ROUTE_KEYS, outs):
        assert o.guards_intact()
        assert o.download().tolist() == ref[key].tolist(), key


def test_route_profile_pins(gpu, oracle):
    """The reference's pinned routing outcomes (tests/oracle.rs:33-89)."""
    lens = [16, 4, 4, 5, 16, 16, 16]
    K = _k().moe_top2_route_f32_t8_e4_k2_c4_v1_gpu.Kernel.load(gpu)

    def run(name):
        outs = [gpu.alloc(n, np.uint32) for n in lens]
        K.prepare(gpu.to_device(np.array(rv.MOE_VECTORS[name], np.float32)), *outs).launch()
        return {k: o.download() for k, o in zip(ROUTE_KEYS, outs)}

    r = run("nominal-balanced")
    assert r["requested_counts"].tolist() == [4, 4, 4, 4]
    assert r["expert_offsets"].tolist() == [0, 4, 8, 12, 16]
    r = run("all-equal-tie-break-and-empty-experts")
    assert r["top2_experts"].tolist() == [0, 1] * 8
    assert r["requested_counts"].tolist() == [8, 8, 0, 0]
    assert r["admitted_counts"].tolist() == [4, 4, 0, 0]
    assert r["expert_offsets"].tolist() == [0, 4, 8, 8, 8]
    assert r["permutation"][8:].tolist() == [0xFFFFFFFF] * 8
    r = run("stable-capacity-overflow")
    assert r["requested_counts"][0] == 8
    assert r["permutation"][:4].tolist() == [0, 2, 4, 6]
    for route in (8, 10, 12, 14):
        assert r["inverse"][route] == 0xFFFFFFFF and r["route_slots"][route] == 0xFFFFFFFF


# ---- router: BASELINE scale ---------------------------------------------------------------

def _route(gpu, logits_dev, tokens, experts, capacity):
    out = {"top2": gpu.alloc(2 * tokens, np.uint32), "requested": gpu.alloc(experts, np.uint32),
           "admitted": gpu.alloc(experts, np.uint32), "offsets": gpu.alloc(experts + 1, np.uint32),
           "slots": gpu.alloc(2 * tokens, np.uint32),
           "permutation": gpu.alloc(2 * tokens, np.uint32),
           "inverse": gpu.alloc(2 * tokens, np.uint32), "weights": gpu.alloc(2 * tokens, np.float32)}
    _k().moe_top2_route(logits_dev, out, tokens, experts, capacity)
    return out


@pytest.mark.parametrize("capacity", [0xFFFFFFFF, 1280, 700, 3])
def test_route_config5_bf16_logits_bit_exact(gpu, oracle, capacity):
    """Config 5 router: 4096 tokens x 8 experts, bf16 logits ~ N(0,1) (seed 5;
    bf16 rounding makes ties frequent, exercising the lower-id rule), at
    unbounded, 1.25x-balanced, tight and tiny capacities."""
    tokens, experts = 4096, 8
    lg = gpu.alloc(tokens * experts, np.uint16)
    _k().fill_normal_bf16(lg, 5, 0x10617, 1.0)
    host_bits = lg.download()
    logits = bf16_to_f32(host_bits)
    out = _route(gpu, lg, tokens, experts, capacity)
    rc, ref = oracle.moe_top2_route(logits, tokens, experts, capacity)
    assert rc == 0
    names = dict(zip(["top2", "requested", "admitted", "offsets", "slots", "permutation",
                      "inverse"], ROUTE_KEYS))
    for mine, theirs in names.items():
        assert_same(out[mine].download(), ref[theirs], mine)
    w = out["weights"].download()
    wref = oracle.moe_top2_weights(logits, tokens, experts, ref["top2_experts"])
    assert np.all(np.abs(w - wref) <= 1e-6 * np.abs(wref))
    assert np.all(w[0::2] + w[1::2] == np.float32(1.0))
    # round trip: permutation and inverse are mutually inverse on admitted routes
    perm, inv = ref["permutation"], ref["inverse"]
    total = ref["expert_offsets"][-1]
    assert all(inv[perm[s]] == s for s in range(total))


@pytest.mark.parametrize("tokens", [1, 255, 256, 257, 1000, 5000])
@pytest.mark.parametrize("experts,capacity", [(2, 0xFFFFFFFF), (7, 100), (64, 3)])
def test_route_workgroup_boundaries(gpu, oracle, tokens, experts, capacity):
    """The slot assignment runs one workgroup per 512 routes: route counts
    below, at and across workgroup boundaries, few and many experts, with
    and without capacity drops; every output array bit-equal to the oracle
    (logits rounded to multiples of 1/4, so ties are frequent)."""
    rng = np.random.default_rng(tokens * 97 + experts)
    logits = (np.round(rng.standard_normal(tokens * experts) * 4) / 4).astype(np.float32)
    out = _route(gpu, gpu.to_device(logits), tokens, experts, capacity)
    rc, ref = oracle.moe_top2_route(logits, tokens, experts, capacity)
    assert rc == 0
    names = dict(zip(["top2", "requested", "admitted", "offsets", "slots", "permutation",
                      "inverse"], ROUTE_KEYS))
    for mine, theirs in names.items():
        assert_same(out[mine].download(), ref[theirs], mine)


@pytest.mark.parametrize("tokens", [4097, 20000, 70001])
@pytest.mark.parametrize("experts,capacity", [(8, 0xFFFFFFFF), (5, 3000), (64, 700)])
def test_route_many_routes_bit_exact(gpu, oracle, tokens, experts, capacity):
    """More than 8192 routes take the count / scan / assign kernels (the
    single kernel's counting grows as routes^2): every output array bit-equal
    to the oracle, with and without capacity drops, ragged last workgroups
    (logits rounded to multiples of 1/4, so ties are frequent)."""
    rng = np.random.default_rng(tokens + experts)
    logits = (np.round(rng.standard_normal(tokens * experts) * 4) / 4).astype(np.float32)
    out = _route(gpu, gpu.to_device(logits), tokens, experts, capacity)
    rc, ref = oracle.moe_top2_route(logits, tokens, experts, capacity)
    assert rc == 0
    names = dict(zip(["top2", "requested", "admitted", "offsets", "slots", "permutation",
                      "inverse"], ROUTE_KEYS))
    for mine, theirs in names.items():
        assert_same(out[mine].download(), ref[theirs], mine)


def test_route_f32_logits_many_experts(gpu, oracle):
    tokens, experts = 1000, 64
    rng = np.random.default_rng(3)
    logits = np.round(rng.standard_normal(tokens * experts) * 4).astype(np.float32)  # many ties
    out = _route(gpu, gpu.to_device(logits), tokens, experts, 40)
    rc, ref = oracle.moe_top2_route(logits, tokens, experts, 40)
    assert rc == 0
    assert_same(out["top2"].download(), ref["top2_experts"], "top2")
    assert_same(out["inverse"].download(), ref["inverse"], "inverse")
    assert_same(out["permutation"].download(), ref["permutation"], "permutation")


# ---- expert combine: exact profile ----------------------------------------------------------

@pytest.mark.parametrize("which", ["equal", "balanced"])
def test_expert_combine_profile_bit_exact(gpu, oracle, which):
    """examples/moe_expert_v1/tests/pipeline_oracle.rs:15-130: the combine of
    the oracle pipeline's compact output, bit-equal."""
    logits = np.array(rv.moe_expert_equal_logits() if which == "equal"
                      else rv.moe_expert_balanced_logits(), np.float32)
    rc, routing = oracle.moe_top2_route(logits, 8, 4, 4)
    assert rc == 0
    acts = rv.moe_expert_activations(oracle.bf16_from_f32)
    weights = rv.moe_expert_weights(oracle.bf16_from_f32)
    rw = rv.moe_expert_route_weights()
    rc, pipe = oracle.moe_expert_pipeline_v1(logits, acts, weights, rw, routing)
    assert rc == 0
    compact = gpu.to_device(pipe["compact_output"])
    out = Guarded(gpu, np.full(128, np.nan, np.float32))
    _k().moe_expert_combine_f32_t8_k2_o16_v1_gpu.Kernel.load(gpu).prepare(
        compact, gpu.to_device(routing["inverse"]), gpu.to_device(rw), out.body).launch()
    assert out.download().view(np.uint32).tolist() == pipe["combined_output"].view(np.uint32).tolist()
    assert out.guards_intact()


# ---- expert FFN ------------------------------------------------------------------------------

def _ffn_case(gpu, oracle, tokens, hidden, ffn, experts, capacity, sample_tokens):
    kern = _k()
    seed = 5
    lg = gpu.alloc(tokens * experts, np.uint16)
    kern.fill_normal_bf16(lg, seed, 0x10617, 1.0)
    x = gpu.alloc(tokens * hidden, np.uint16)
    kern.fill_normal_bf16(x, seed, 0xAC7, 1.0)
    wsz = experts * ffn * hidden
    wg, wu, wd = (gpu.alloc(wsz, np.uint16) for _ in range(3))
    kern.fill_normal_bf16(wg, seed, 0x6A7E, 0.02)
    kern.fill_normal_bf16(wu, seed, 0x0B0B, 0.02)
    kern.fill_normal_bf16(wd, seed, 0xD0D0, 0.02)
    routing = _route(gpu, lg, tokens, experts, capacity)
    ws = gpu.alloc(kern.moe_ffn_workspace_bytes(tokens, hidden, ffn, experts), np.uint8)
    out = Guarded(gpu, np.full(tokens * hidden, 0x7FDE, np.uint16))
    kern.moe_ffn_top2(x, wg, wu, wd, routing, out.body, ws, tokens, hidden, ffn, experts)
    assert out.guards_intact()
    got = bf16_to_f32(out.download()).reshape(tokens, hidden)
    top2 = routing["top2"].download()
    inv = routing["inverse"].download()
    w = routing["weights"].download()
    xs = x.download().reshape(tokens, hidden)
    if callable(sample_tokens):
        sample_tokens = sample_tokens(routing["offsets"].download(),
                                      routing["permutation"].download())
    toks = np.array(list(sample_tokens), np.int64)
    hw = [t.download() for t in (wg, wu, wd)]
    pairs = [(int(t), 2 * int(t) + rank) for t in toks for rank in range(2)
             if inv[2 * int(t) + rank] != 0xFFFFFFFF]
    y = oracle.moe_ffn_routes(xs, hw[0], hw[1], hw[2], hidden, ffn,
                              np.array([p[0] for p in pairs], np.uint32),
                              np.array([top2[p[1]] for p in pairs], np.uint32))
    refs = {int(t): np.zeros(hidden, np.float32) for t in toks}
    for (t, r), yr in zip(pairs, y):  # +0, then each admitted rank in order
        refs[t] = refs[t] + np.float32(w[r]) * yr
    worst = max(rel_err(got[t], refs[int(t)]) for t in toks)
    return worst, inv


def test_moe_ffn_small_all_tokens(gpu, oracle):
    tokens, hidden, ffn, experts = 256, 256, 512, 8
    worst, inv = _ffn_case(gpu, oracle, tokens, hidden, ffn, experts, 0xFFFFFFFF, range(tokens))
    assert worst <= 1e-2, worst


@pytest.mark.parametrize("experts", [2, 3])
def test_moe_ffn_few_experts(gpu, oracle, experts):
    """Two and three experts: the expert halves that run on the caller's
    stream and on the side stream are 1 + 1 and 1 + 2 experts."""
    tokens, hidden, ffn = 256, 256, 256
    worst, _ = _ffn_case(gpu, oracle, tokens, hidden, ffn, experts, 0xFFFFFFFF, range(tokens))
    assert worst <= 1e-2, worst


@pytest.mark.parametrize("ffn", [384, 640])
def test_moe_ffn_odd_128_blocks(gpu, oracle, ffn):
    """ffn an odd multiple of 128 (the smallest granule the entry point
    admits): an odd number of 128-wide gate/up blocks, and down-projection
    k-halves of 192 or 320, an odd number of 64-k pipeline stages."""
    tokens, hidden, experts = 300, 256, 4
    worst, _ = _ffn_case(gpu, oracle, tokens, hidden, ffn, experts, 0xFFFFFFFF, range(tokens))
    assert worst <= 1e-2, worst


def test_moe_ffn_garbage_routing_stays_in_bounds(gpu, oracle):
    """Routing arrays that fail the consistency check (random offsets, some
    decreasing or beyond 2*tokens; permutation and inverse entries out of
    range) give unspecified outputs, but every access stays inside the
    caller's buffers: the output and workspace guards stay intact and the
    inputs unchanged.  (Bounds of the tile list for any offsets are shown on
    the CPU by tests/test_moe_tiles.py.)"""
    kern = _k()
    tokens, hidden, ffn, experts = 200, 256, 256, 8
    rng = np.random.default_rng(17)
    routes = 2 * tokens
    x = Guarded(gpu, oracle.bf16_from_f32(rng.standard_normal(tokens * hidden)))
    w = [Guarded(gpu, oracle.bf16_from_f32(rng.standard_normal(experts * ffn * hidden) * 0.02))
         for _ in range(3)]
    wsb = kern.moe_ffn_workspace_bytes(tokens, hidden, ffn, experts)
    for trial in range(6):
        offsets = rng.integers(0, routes + 300, experts + 1).astype(np.uint32)
        if trial % 2:
            offsets = np.sort(offsets)
        routing = {
            "top2": Guarded(gpu, rng.integers(0, 2**32, routes, dtype=np.uint64).astype(np.uint32)),
            "offsets": Guarded(gpu, offsets),
            "permutation": Guarded(gpu, rng.integers(0, routes + 50, routes).astype(np.uint32)),
            "inverse": Guarded(gpu, rng.integers(0, routes + 50, routes).astype(np.uint32)),
            "weights": Guarded(gpu, rng.random(routes).astype(np.float32)),
        }
        out = Guarded(gpu, np.full(tokens * hidden, 0x7FDE, np.uint16))
        ws = Guarded(gpu, np.zeros(wsb, np.uint8))
        kern.moe_ffn_top2(x.body, w[0].body, w[1].body, w[2].body,
                          {k: v.body for k, v in routing.items()}, out.body, ws.body, tokens,
                          hidden, ffn, experts)
        assert out.guards_intact() and ws.guards_intact(), trial
        assert x.unchanged() and all(t.unchanged() for t in w)
        assert all(v.unchanged() for v in routing.values())


@pytest.mark.parametrize("hidden,ffn", [(256, 384), (512, 256)])
def test_moe_ffn_every_short_tile_path(gpu, oracle, hidden, ffn):
    """A routing built by hand (every route admitted, slots in route order
    per expert) whose expert row counts put tiles on every A-tile form: the
    short form (at most 64 rows: 5, 31, 32, 33, 64) and A tiles of 96 (65),
    128 (128), 160 (129, both tiles of 289 and of 300, the second of 321),
    192 (the first of 321, both of 384), 224 (200, both of 418), 256 (256)
    and 288 rows (257, whose ninth row block accumulates in VGPRs); every
    token's output against the oracle."""
    kern = _k()
    counts = [5, 31, 32, 33, 64, 65, 128, 129, 200, 256, 257, 300, 289, 321, 384, 418]
    experts = len(counts)
    routes = sum(counts)
    assert routes % 2 == 0
    tokens = routes // 2
    rng = np.random.default_rng(hidden + ffn)
    top2 = np.repeat(np.arange(experts, dtype=np.uint32), counts)
    rng.shuffle(top2)
    order = np.argsort(top2, kind="stable")
    perm = order.astype(np.uint32)
    inv = np.empty(routes, np.uint32)
    inv[order] = np.arange(routes, dtype=np.uint32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.uint32)
    w0 = rng.uniform(0.5, 1.0, tokens).astype(np.float32)
    weights = np.stack([w0, np.float32(1.0) - w0], axis=1).ravel()
    x = oracle.bf16_from_f32(rng.standard_normal(tokens * hidden)).reshape(tokens, hidden)
    wsz = experts * ffn * hidden
    wg, wu, wd = (oracle.bf16_from_f32(rng.standard_normal(wsz) * 0.05) for _ in range(3))
    routing = {"top2": gpu.to_device(top2), "offsets": gpu.to_device(offsets),
               "permutation": gpu.to_device(perm), "inverse": gpu.to_device(inv),
               "weights": gpu.to_device(weights)}
    ws = gpu.alloc(kern.moe_ffn_workspace_bytes(tokens, hidden, ffn, experts), np.uint8)
    out = Guarded(gpu, np.full(tokens * hidden, 0x7FDE, np.uint16))
    kern.moe_ffn_top2(gpu.to_device(x), gpu.to_device(wg), gpu.to_device(wu), gpu.to_device(wd),
                      routing, out.body, ws, tokens, hidden, ffn, experts)
    assert out.guards_intact()
    got = bf16_to_f32(out.download()).reshape(tokens, hidden)
    y = oracle.moe_ffn_routes(x, wg, wu, wd, hidden, ffn,
                              np.arange(routes, dtype=np.uint32) // 2, top2)
    want = np.zeros((tokens, hidden), np.float32)
    for rank in range(2):
        want = want + weights.reshape(tokens, 2)[:, rank][:, None] * y[rank::2]
    assert rel_err(got, want) <= 1e-2
    # every token within one bf16 rounding of its own reference row scale
    scale = np.max(np.abs(want), axis=1, keepdims=True)
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * scale + 1e-6)


def test_moe_ffn_small_with_drops(gpu, oracle):
    """Capacity below demand: dropped routes contribute nothing."""
    tokens, hidden, ffn, experts = 256, 256, 256, 8
    worst, inv = _ffn_case(gpu, oracle, tokens, hidden, ffn, experts, 40, range(tokens))
    assert (inv == 0xFFFFFFFF).any()
    assert worst <= 1e-2, worst


def test_moe_ffn_whole_k_down(gpu, oracle):
    """1200 tokens, hidden 4096, 8 experts: an even routing would give 16
    m-tiles of 16 n-blocks, exactly one round of 256 down tiles over K
    whole, which the entry point then prefers to two rounds of half-K tiles
    (the smaller FFN tests run split K); the first and last 8 slots of every
    expert against the oracle."""
    tokens, hidden, ffn, experts = 1200, 4096, 512, 8
    worst, _ = _ffn_case(gpu, oracle, tokens, hidden, ffn, experts, 0xFFFFFFFF,
                         _per_expert_tokens(8))
    assert worst <= 1e-2, worst


def _tail_tokens(offsets, permutation):
    """Tokens routed to the rows around the 256-row mark and around row 160
    of every expert over 256 rows, plus each expert's first and last rows.
    An expert of 257-300 rows, which once ran as a full tile and a remainder
    of at most 44 rows, runs as one 288-row tile (up to 288 rows) or as two
    tiles of 160 and 129-140 rows; the picked rows include the last rows of
    each."""
    rows = set()
    split = 0
    for e in range(len(offsets) - 1):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi - lo > 256:
            split += 1
            rows.update(range(lo + 248, hi))
            rows.update(range(lo + 120, lo + 168))  # around the balanced boundary
        rows.update(range(lo, min(hi, lo + 4)))
        rows.update(range(max(lo, hi - 4), hi))
    assert split >= 2, split
    return sorted({int(permutation[r]) >> 1 for r in rows if r < int(offsets[-1])})


def test_moe_ffn_short_last_tiles(gpu, oracle):
    """Experts of about 275 rows (one 288-row tile, or two of 160 and
    129-140 rows past 288): every token routed into the rows around the
    256-row mark and the two-tile boundary is checked, with each expert's
    first and last rows."""
    tokens, hidden, ffn, experts = 1100, 512, 1024, 8
    worst, _ = _ffn_case(gpu, oracle, tokens, hidden, ffn, experts, 0xFFFFFFFF, _tail_tokens)
    assert worst <= 1e-2, worst


def _per_expert_tokens(per):
    """Tokens of the first `per` slots of every expert plus those of its last
    `per` slots (so each expert's first and last m-tiles are covered)."""
    def pick(offsets, permutation):
        rows = set()
        for e in range(len(offsets) - 1):
            lo, hi = int(offsets[e]), int(offsets[e + 1])
            rows.update(range(lo, min(hi, lo + per)))
            rows.update(range(max(lo, hi - per), hi))
        return sorted({int(permutation[r]) >> 1 for r in rows})
    return pick


def test_moe_ffn_config5_sampled_tokens(gpu, oracle):
    """4096 tokens, hidden 4096, 8 experts, FFN 14336,
    weights N(0, 0.02), unbounded capacity; the tokens of the first 64 and
    the last 64 slots of every expert (both routes of each) end to end."""
    worst, _ = _ffn_case(gpu, oracle, 4096, 4096, 14336, 8, 0xFFFFFFFF, _per_expert_tokens(64))
    assert worst <= 1e-2, worst


def test_moe_ffn_token_matrix_past_2gib(gpu, oracle):
    """A token matrix of 2^31 bytes or more does not fit one 32-bit buffer
    resource, so the gate/up tiles read rows gathered into the workspace
    (gather_kernel, gate_up_kernel<false>) instead of the token rows in place
    through the permutation: 2^22 tokens of hidden 256, FFN 128, 2 experts
    (x is 2 GiB, the workspace 22 GiB); the tokens of the first and last 64
    slots of each expert end to end."""
    worst, _ = _ffn_case(gpu, oracle, 1 << 22, 256, 128, 2, 0xFFFFFFFF, _per_expert_tokens(64))
    assert worst <= 1e-2, worst


# ---- fp8 ------------------------------------------------------------------------------------

def _edge_values():
    v = [0.0, -0.0, 448.0, -448.0, 449.0, 463.99, 464.0, 464.01, 479.0, 480.0, 1e30, -1e30,
         float("inf"), float("-inf"), 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -11, 2.0 ** -6,
         2.0 ** -6 * 1.0625, 2.0 ** -6 * 0.9375, 1.0625, 1.1875, 0.5 + 2.0 ** -5, 240.0, 1e-45,
         -1e-40, 2.0 ** -7 * 15 / 16]
    return np.array(v, np.float32)


def test_e4m3_encoding_bit_exact(gpu, oracle):
    """Device RNE/satfinite encoding equals the oracle's OCP closed form on
    every bf16-representable value, edge cases and random f32 values."""
    allbf = bf16_to_f32(np.arange(65536, dtype=np.uint16))
    allbf = allbf[~np.isnan(allbf)]
    rng = np.random.default_rng(0)
    rand = (rng.standard_normal(1 << 20) * rng.choice([1e-3, 1.0, 30.0, 1000.0], 1 << 20)).astype(np.float32)
    x = np.concatenate([allbf, _edge_values(), rand]).astype(np.float32)
    x = np.concatenate([x, np.zeros((-x.size) % 4, np.float32)])
    kern = _k()
    dx = gpu.to_device(x)
    one = gpu.to_device(np.array([1.0], np.float32))
    dq = gpu.alloc(x.size, np.uint8)
    kern.quantize_e4m3(dx, one, dq)
    got = dq.download()
    ref = oracle.quantize_e4m3(x, 1.0)
    assert_same(got, ref, "e4m3 codes")


def test_amax_scale_and_quantize_bit_exact(gpu, oracle):
    kern = _k()
    n = 1_000_003
    xh = oracle.fill_normal_f32(n, 4, 0xA8A8, 1.0)
    x = gpu.to_device(xh)
    amax = gpu.alloc(1, np.float32)
    scale = gpu.alloc(1, np.float32)
    kern.amax_f32(x, amax)
    kern.fp8_scale_from_amax(amax, scale)
    a_ref = oracle.amax_f32(xh)
    assert amax.download()[0] == np.float32(a_ref)
    s_ref = np.float32(np.float32(a_ref) / np.float32(448.0))
    assert scale.download()[0] == s_ref
    q = gpu.alloc(n, np.uint8)
    kern.quantize_e4m3(x, scale, q)
    assert_same(q.download(), oracle.quantize_e4m3(xh, float(s_ref)), "quantized")


def _fp8_case(gpu, oracle, m, n, k, points, block=None):
    """rel-err of the device GEMM at `points` (rows, cols); the outputs of
    whole rows block[0]..block[1]-1 among them come from the row-block form
    of the oracle, the rest from the per-point form."""
    kern = _k()
    a32 = gpu.alloc(m * k, np.float32)
    b32 = gpu.alloc(n * k, np.float32)
    kern.fill_normal_f32(a32, 4, 0xA, 1.0)
    kern.fill_normal_f32(b32, 4, 0xB, 1.0)
    sa, sb, am = gpu.alloc(1, np.float32), gpu.alloc(1, np.float32), gpu.alloc(1, np.float32)
    aq, bq = gpu.alloc(m * k, np.uint8), gpu.alloc(n * k, np.uint8)
    for src, s, q in ((a32, sa, aq), (b32, sb, bq)):
        kern.amax_f32(src, am)
        kern.fp8_scale_from_amax(am, s)
        kern.quantize_e4m3(src, s, q)
    c = Guarded(gpu, np.full(m * n, 0x7FDE, np.uint16))
    kern.gemm_fp8_nt(aq, bq, sa, sb, c.body, m, n, k)
    assert c.guards_intact()
    got = bf16_to_f32(c.download()).reshape(m, n)
    ah, bh = aq.download().reshape(m, k), bq.download().reshape(n, k)
    sab = float(np.float32(sa.download()[0] * sb.download()[0]))
    rows, cols = points
    if block is None:
        ref_f32, _ = oracle.gemm_fp8_points(k, ah[rows], bh[cols], sab)
        return rel_err(got[rows, cols], ref_f32)
    inb = (rows >= block[0]) & (rows < block[1])
    ref_blk = oracle.gemm_fp8_nt_rows(n, k, ah, bh, sab, block[0], block[1])
    ref_pts, _ = oracle.gemm_fp8_points(k, ah[rows[~inb]], bh[cols[~inb]], sab)
    got_all = np.concatenate([got[rows[~inb], cols[~inb]], got[rows[inb], cols[inb]]])
    ref_all = np.concatenate([ref_pts, ref_blk[rows[inb] - block[0], cols[inb]]])
    return rel_err(got_all, ref_all)


@pytest.mark.parametrize("m,n,k", [(256, 256, 128), (512, 768, 1024), (256, 512, 4096),
                                   (256, 256, 384)])
def test_gemm_fp8_all_outputs(gpu, oracle, m, n, k):
    rr, cc = np.meshgrid(np.arange(m), np.arange(n), indexing="ij")
    assert _fp8_case(gpu, oracle, m, n, k, (rr.ravel(), cc.ravel())) <= 1e-2


# any M, N: edge tiles on the fast path (K a multiple of 16, the last stage
# partial when K is not a multiple of 128), the generic bounds-checked kernel
# otherwise (E4M3 widened exactly to bf16)
@pytest.mark.parametrize("m,n,k", [(300, 520, 256), (1, 257, 128), (257, 256, 384),
                                   (100, 70, 96), (33, 65, 200), (256, 256, 160), (5, 3, 1)])
def test_gemm_fp8_any_shape(gpu, oracle, m, n, k):
    rr, cc = np.meshgrid(np.arange(m), np.arange(n), indexing="ij")
    assert _fp8_case(gpu, oracle, m, n, k, (rr.ravel(), cc.ravel())) <= 1e-2


# K a multiple of 16 but not of 128: the pipelined tiles with a partial last
# stage (its chunks past K load zeros) on the 128x128 form (three and two
# stages), the 256x256 tile and its tail round
@pytest.mark.parametrize("m,n,k", [(256, 256, 16), (512, 768, 208), (300, 520, 272),
                                   (4096, 2048, 144), (6144, 6144, 48)])
def test_gemm_fp8_k_tail(gpu, oracle, m, n, k):
    rng = np.random.default_rng(m + n + k)
    if m * n <= 400_000:
        rr, cc = np.meshgrid(np.arange(m), np.arange(n), indexing="ij")
        points = (rr.ravel(), cc.ravel())
    else:
        rows = np.concatenate([np.arange(0, m, 128), rng.integers(0, m, 4000), [m - 1]])
        points = (rows, rng.integers(0, n, rows.size))
    assert _fp8_case(gpu, oracle, m, n, k, points) <= 1e-2


@pytest.mark.parametrize("m,n,k,kp", [(1024, 1024, 4000, 4096), (300, 520, 208, 256),
                                      (6144, 6144, 80, 128), (512, 384, 1001, 1008),
                                      (300, 520, 77, 80)])
def test_gemm_fp8_k_tail_matches_zero_padded_k(gpu, m, n, k, kp):
    """K not a multiple of 128 against the same operands zero-padded to whole
    stages (the plain tiles): the partial stage's zero chunks are exactly the
    padding and the scales are the same, so C is bit-identical.  K not a
    multiple of 16 (1001, 77): the rows are first repacked into scratch rows
    of K rounded up to 16, which is the padded operand itself."""
    kern = _k()
    rng = np.random.default_rng(k)
    # E4M3 codes without the NaN pair (0x7F, 0xFF)
    a = rng.integers(0, 0x7F, (m, k), dtype=np.uint8) | (rng.integers(0, 2, (m, k), dtype=np.uint8) << 7)
    b = rng.integers(0, 0x7F, (n, k), dtype=np.uint8) | (rng.integers(0, 2, (n, k), dtype=np.uint8) << 7)
    ap = np.zeros((m, kp), np.uint8)
    bp = np.zeros((n, kp), np.uint8)
    ap[:, :k], bp[:, :k] = a, b
    sa = gpu.to_device(np.array([1.0 / 64], np.float32))
    sb = gpu.to_device(np.array([1.0 / 32], np.float32))
    c, cp = gpu.alloc(m * n, np.uint16), gpu.alloc(m * n, np.uint16)
    kern.gemm_fp8_nt(gpu.to_device(a.ravel()), gpu.to_device(b.ravel()), sa, sb, c, m, n, k)
    kern.gemm_fp8_nt(gpu.to_device(ap.ravel()), gpu.to_device(bp.ravel()), sa, sb, cp, m, n, kp)
    assert_same(c.download(), cp.download(), f"K {k} vs zero-padded K {kp}")


@pytest.mark.parametrize("m,n,k,which", [(512, 384, 1024, "a"), (384, 640, 4096, "b"),
                                         (256, 256, 208, "ab")])
def test_gemm_fp8_misaligned_operands_match_aligned(gpu, m, n, k, which):
    """A and/or B one byte past a 16-byte boundary: their rows are copied
    into aligned scratch and the pipelined tile runs on the copies, so C is
    bit-identical to the aligned operands' (inputs unchanged)."""
    kern = _k()
    rng = np.random.default_rng(m + k)
    a = rng.integers(0, 0x7F, m * k, dtype=np.uint8) | (rng.integers(0, 2, m * k, dtype=np.uint8) << 7)
    b = rng.integers(0, 0x7F, n * k, dtype=np.uint8) | (rng.integers(0, 2, n * k, dtype=np.uint8) << 7)
    sa = gpu.to_device(np.array([1.0 / 64], np.float32))
    sb = gpu.to_device(np.array([1.0 / 32], np.float32))
    want = gpu.alloc(m * n, np.uint16)
    kern.gemm_fp8_nt(gpu.to_device(a), gpu.to_device(b), sa, sb, want, m, n, k)
    offs = {key: Guarded(gpu, np.concatenate([np.zeros(1, np.uint8), host]))
            for key, host in (("a", a), ("b", b)) if key in which}
    ga = offs["a"].full.view(GUARD + 1, m * k) if "a" in offs else gpu.to_device(a)
    gb = offs["b"].full.view(GUARD + 1, n * k) if "b" in offs else gpu.to_device(b)
    got = Guarded(gpu, np.full(m * n, 0x7FDE, np.uint16))
    kern.gemm_fp8_nt(ga, gb, sa, sb, got.body, m, n, k)
    assert got.guards_intact() and all(o.unchanged() for o in offs.values())
    assert_same(got.download(), want.download(), f"{which} at a 1-byte offset vs aligned")


@pytest.mark.parametrize("m,n,k", [(4096, 2048, 128), (4000, 2000, 256)])
def test_gemm_fp8_small_grid_two_stage(gpu, oracle, m, n, k):
    """128 tiles of 256x256 (512 small tiles: the two-stage 128x128 form),
    whole and edge: sampled outputs of every tile row against the oracle."""
    rng = np.random.default_rng(m + n + k)
    rows = np.concatenate([np.arange(0, m, 128), rng.integers(0, m, 4000)])
    cols = rng.integers(0, n, rows.size)
    assert _fp8_case(gpu, oracle, m, n, k, (rows, cols)) <= 1e-2


def test_gemm_fp8_small_grid_matches_large_tiles(gpu):
    """The same 2048 rows of A against the same B: at M = 2048 (64 tiles of
    256x256, so 128x128 tiles run) and inside M = 4352 (136 tiles, the
    256x256 tile), on whole and edge shapes: every output gets the same MFMAs
    in the same k order and the same scale, so the rows are bit-identical."""
    kern = _k()
    for n, k in ((2048, 512), (2000, 384)):
        big = 4352
        a32 = gpu.alloc(big * k, np.float32)
        b32 = gpu.alloc(n * k, np.float32)
        kern.fill_normal_f32(a32, 9, 0xA, 1.0)
        kern.fill_normal_f32(b32, 9, 0xB, 1.0)
        sa, sb, am = gpu.alloc(1, np.float32), gpu.alloc(1, np.float32), gpu.alloc(1, np.float32)
        aq, bq = gpu.alloc(big * k, np.uint8), gpu.alloc(n * k, np.uint8)
        for src, s_, q in ((a32, sa, aq), (b32, sb, bq)):
            kern.amax_f32(src, am)
            kern.fp8_scale_from_amax(am, s_)
            kern.quantize_e4m3(src, s_, q)
        c_big = gpu.alloc(big * n, np.uint16)
        kern.gemm_fp8_nt(aq, bq, sa, sb, c_big, big, n, k)
        c_small = gpu.alloc(2048 * n, np.uint16)
        kern.gemm_fp8_nt(aq.view(0, 2048 * k), bq, sa, sb, c_small, 2048, n, k)
        assert_same(c_small.download(), c_big.download()[:2048 * n], f"n={n} k={k}")


def test_gemm_fp8_k0_writes_positive_zero(gpu):
    kern = _k()
    one = gpu.to_device(np.array([1.0], np.float32))
    empty = gpu.alloc(0, np.uint8)
    c = Guarded(gpu, np.full(7 * 9, 0xFFFF, np.uint16))
    kern.gemm_fp8_nt(empty, empty, one, one, c.body, 7, 9, 0)
    assert c.guards_intact() and c.download().tolist() == [0] * 63


def test_gemm_fp8_config4_sampled(gpu, oracle):
    """8192^3 e4m3 with amax/448 per-tensor scales; one
    whole 128-row block (rows 4096..4223, all 8192 columns: 1M outputs at
    full K) plus 4096 random outputs."""
    m = n = k = 8192
    rng = np.random.default_rng(4)
    rr, cc = np.meshgrid(np.arange(4096, 4096 + 128), np.arange(n), indexing="ij")
    rows = np.concatenate([rng.integers(0, m, 4096), rr.ravel()])
    cols = np.concatenate([rng.integers(0, n, 4096), cc.ravel()])
    assert _fp8_case(gpu, oracle, m, n, k, (rows, cols), block=(4096, 4096 + 128)) <= 1e-2


def test_gemm_fp8_staged_epilogue(gpu, oracle):
    """Operands of 192 MiB, the size from which C leaves through LDS with
    nontemporal stores: four rows over the first four column tiles plus 4096
    random outputs."""
    m, n, k = 256, 24576, 8192
    rng = np.random.default_rng(5)
    full = np.array([0, 97, 130, 255])
    rows = np.concatenate([np.repeat(full, 1024), rng.integers(0, m, 4096)])
    cols = np.concatenate([np.tile(np.arange(1024), len(full)), rng.integers(0, n, 4096)])
    assert _fp8_case(gpu, oracle, m, n, k, (rows, cols)) <= 1e-2
