"""Routing bit-exact by construction: near ties.

The reference sums each router logit sequentially in fp32
(src/cpu/reference_ops.cpp:85-93) and ranks by softmax probability with the
lower id first among equals (:130-212). The device sums in other orders, so
two logits closer than its rounding difference (about 1e-6 at the
Qwen3-Next shape) could come out in either order. Each device logit carries a
bound on its distance from the reference's; a selection whose order the
bounds do not prove recomputes its candidates in the reference's order.

These routers are built so that several pairs of experts -- the top two, two
in the middle of the picks, the k-th against an expert outside -- have
logits about 7e-7..1e-6 apart for the token under test (the reference's own
rounding moves each gap by a few 1e-7), with the higher logit sometimes on
the higher id. Every path must give the oracle's ids bit for bit, and the
routing counters must show the exact path ran.
"""

import numpy as np
import pytest

import oracle as O
import osm_hip
from helpers import bf16_bits, bf16_to_f32, random_blob
from test_gpu_moe import assert_weights

pytestmark = pytest.mark.gpu

D, I, G, E, K = 2048, 128, 64, 512, 10


def _bf16_next(bits):
    """The bf16 value one ulp away from zero (same sign)."""
    return np.uint16(int(bits) + 1)


def near_tie_router(rng, x_route, dtype, gap=(7e-7, 1e-6)):
    """A router [E, D] (f32 values, or bf16 bits) with near ties for input
    x_route (what the router multiplies: x, or RMSNorm(x)): five copies of
    picked rows, each with one element moved so its logit lands `gap` above
    or below the original's."""
    lo, hi = gap
    w = rng.normal(0, 0.02, (E, D)).astype(np.float32)
    if dtype == osm_hip.BF16:
        bits = bf16_bits(w)
        w = bf16_to_f32(bits)
    logits = w.astype(np.float64) @ x_route.astype(np.float64)
    order = np.argsort(-logits, kind="stable")
    # (source rank, copy target, side): the copy gets the source's row with
    # one element nudged.
    plan = [(0, int(order[200]), +1), (4, int(order[300]), -1), (K - 1, int(order[400]), +1),
            (K - 1, int(order[401]), -1), (6, int(order[450]), +1)]
    for src_rank, dst, sign in plan:
        src = int(order[src_rank])
        row = w[src].copy()
        rb = bits[src].copy() if dtype == osm_hip.BF16 else None
        # A column where one step of the weight moves the logit by lo..hi.
        for c in rng.permutation(D):
            if dtype == osm_hip.BF16:
                nb = _bf16_next(rb[c])
                step = float(bf16_to_f32(np.array([nb], np.uint16))[0] - row[c])
            else:
                step = 0.5 * (lo + hi) / max(abs(float(x_route[c])), 1e-3) * np.sign(float(x_route[c]) or 1.0)
            delta = step * float(x_route[c])
            if lo <= abs(delta) <= hi:
                break
        else:
            raise AssertionError("no column gives the requested gap")
        # Nudge in the direction `sign` asks for.
        if dtype == osm_hip.BF16:
            if np.sign(delta) == sign:
                rb[c] = _bf16_next(rb[c])
            else:
                rb[c] = np.uint16(int(rb[c]) - 1) if (int(rb[c]) & 0x7FFF) else rb[c]
            bits[dst] = rb
            w[dst] = bf16_to_f32(rb)
        else:
            row[c] = np.float32(row[c] + (step if np.sign(delta) == sign else -step))
            w[dst] = row
    return (bits if dtype == osm_hip.BF16 else w), w


@pytest.mark.parametrize("dtype,sublayer", [(osm_hip.F32, False), (osm_hip.BF16, False), (osm_hip.BF16, True)])
def test_near_ties_every_path(ctx, dtype, sublayer):
    rng = np.random.default_rng(7 + dtype + (10 if sublayer else 0))
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    blob = random_blob(rng, D, I, G, O.META_BF16)[0]  # one blob everywhere: routing is under test
    slab = osm_hip.ExpertSlab(ctx, g, 1, E)
    for e in range(E):
        slab.upload(0, e, blob)
    x = rng.normal(0, 1, D).astype(np.float32)
    norm = (1.0 + rng.normal(0, 0.02, D)).astype(np.float32) if sublayer else None
    x_route = O.rms_norm(x, 1, D, norm, 1e-6) if sublayer else x
    router, router_f = near_tie_router(rng, x_route, dtype)
    ora = O.route_qwen_top_k(x_route, router_f, D, E, K, True)
    lg = np.sort(ora["logits"])[::-1]
    assert np.sum(np.abs(np.diff(lg[:K + 1])) < 1e-6) >= 2  # the near ties are there
    moe = osm_hip.MoeLayer(ctx, g, E, K, router, dtype, norm_weight=norm, max_tokens=24)

    # One token (selection inside gate/up), 16 tokens (the select kernel),
    # grouped at 16 (the per-token router) and 24 (the router GEMM), each
    # token the same x.
    for path, T in [(osm_hip.PATH_PER_TOKEN, 1), (osm_hip.PATH_PER_TOKEN, 16), (osm_hip.PATH_GROUPED, 16),
                    (osm_hip.PATH_GROUPED, 24)]:
        moe.routing_stats(reset=True)
        moe.set_path(path)
        xs = np.tile(x, (T, 1))
        gpu = moe.run_slab(slab, 0, xs, sublayer=sublayer)
        for t in range(T):
            assert np.array_equal(gpu["ids"][t], ora["ids"]), (path, T, t, list(gpu["ids"][t]), list(ora["ids"]))
            assert_weights(gpu["weights"][t], gpu["logits"][t], gpu["ids"][t], ora["weights"], ora["logits"])
        st = moe.routing_stats()
        assert st["selections"] == T, (path, T, st)
        assert st["exact"] == T, (path, T, st)  # every copy of the token needed the exact path


def test_far_apart_logits_take_the_fast_path(ctx):
    # The Qwen3-Next-shaped seeded layer: ordinary tokens are proven by the
    # bounds and never need the exact path, except rarely.
    from test_gpu_moe import QwenLayer
    L = QwenLayer(ctx, 91, max_tokens=64)
    x = O.synth_tokens(91, 0, 64, L.D)
    L.moe.routing_stats(reset=True)
    L.moe.set_path(osm_hip.PATH_PER_TOKEN)
    gpu = L.moe.run_slab(L.slab, 0, x)
    st = L.moe.routing_stats()
    assert st["selections"] == 64 and st["exact"] <= 12, st
    router = O.bf16_bits_to_f32(L.router_bits)
    for t in range(64):
        ora = O.route_qwen_top_k(x[t], router, L.D, L.E, L.k, True)
        assert np.array_equal(gpu["ids"][t], ora["ids"]), t


def test_ties_within_exp_rounding_are_counted(ctx):
    # Logits 2.5e-7..4.5e-7 apart (one or two ulps of a logit near 2): their
    # exps are within a few ulps, where the
    # reference's order also rests on the last bit of its exp and on how the
    # division by the softmax sum rounds. The selection still ranks them by
    # the exp of the reference's logits (here the oracle's order) and counts
    # each such adjacent pair.
    rng = np.random.default_rng(5)
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    blob = random_blob(rng, D, I, G, O.META_BF16)[0]
    slab = osm_hip.ExpertSlab(ctx, g, 1, E)
    for e in range(E):
        slab.upload(0, e, blob)
    x = rng.normal(0, 1, D).astype(np.float32)
    router, router_f = near_tie_router(rng, x, osm_hip.F32, gap=(2.5e-7, 4.5e-7))
    ora = O.route_qwen_top_k(x, router_f, D, E, K, True)
    moe = osm_hip.MoeLayer(ctx, g, E, K, router, osm_hip.F32, max_tokens=1)
    gpu = moe.run_slab(slab, 0, x[None, :])
    assert np.array_equal(gpu["ids"][0], ora["ids"]), (list(gpu["ids"][0]), list(ora["ids"]))
    st = moe.routing_stats()
    assert st["exact"] == 1 and st["unresolved"] >= 1, st


def test_router_gemm_bounds_prove_most_tokens(ctx):
    # The grouped path's router GEMM bounds its logits too (per-step MFMA
    # sums, 32-column norms): most tokens of a 128-token bf16 chunk are
    # proven without the exact path, and every token's ids are the oracle's.
    from test_gpu_moe import QwenLayer
    T = 128
    L = QwenLayer(ctx, 92, max_tokens=T)
    xf = O.synth_tokens(92, 7000, T, L.D)
    bits = ((xf.view(np.uint32) + 0x7FFF + ((xf.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    xw = (bits.astype(np.uint32) << 16).view(np.float32)
    xb, y = ctx.alloc(T * L.D * 2), ctx.alloc(T * L.D * 4)
    xb.upload(bits)
    L.moe.routing_stats(reset=True)
    L.moe.prefill_device(L.slab, 0, xb.ptr, y.ptr, T)
    routing = L.moe.routing(T)
    st = L.moe.routing_stats()
    assert st["selections"] == T and st["exact"] <= T // 3, st
    router = O.bf16_bits_to_f32(L.router_bits)
    for t in range(T):
        ora = O.route_qwen_top_k(xw[t], router, L.D, L.E, L.k, True)
        assert np.array_equal(routing["ids"][t], ora["ids"]), t
