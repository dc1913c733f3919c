"""The one-token decode as a single launch: router, selection, gate/up and
down workgroups of one grid that signal each other through counters.

It runs the same per-phase code as the three per-token kernels, so the bar
against them is bit-equality of every output (ids, weights, mass, logits,
shared gate, normalised input, y); against the oracle the decode bars hold
(ids bit-exact, weights and shared gate within 1e-6, y within 1e-3 relative
L2). Every test also checks that no wait of any launch ran out of spins."""

import numpy as np
import pytest

import oracle as O
import osm_hip
from helpers import max_abs, random_blob, rel_l2
from test_gpu_moe import QwenLayer, assert_token_parity

pytestmark = pytest.mark.gpu

FIELDS = ("ids", "weights", "mass", "logits", "shared_gate", "out")


def bf16_bits(a):
    u = np.asarray(a, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def both_paths(moe, slab, x, sublayer=False):
    moe.set_path(osm_hip.PATH_SINGLE_LAUNCH)
    one = moe.run_slab(slab, 0, x, sublayer=sublayer)
    moe.set_path(osm_hip.PATH_PER_TOKEN)
    three = moe.run_slab(slab, 0, x, sublayer=sublayer)
    return one, three


def assert_same_bits(one, three, sublayer=False):
    for f in FIELDS + (("normalized",) if sublayer else ()):
        if f in one:
            assert np.array_equal(one[f], three[f]), f


@pytest.mark.parametrize("sublayer", [False, True])
def test_single_launch_qwen_shape(ctx, sublayer):
    seed = 61 + int(sublayer)
    L = QwenLayer(ctx, seed, max_tokens=1, norm=sublayer)
    xs = O.synth_tokens(seed, 500, 6, L.D) * np.float32(2.0 if sublayer else 1.0)
    for t in range(6):
        one, three = both_paths(L.moe, L.slab, xs[t:t + 1], sublayer)
        assert_same_bits(one, three, sublayer)
        if t < 2:
            assert_token_parity(one, 0, L.oracle_token(xs[t], sublayer=sublayer), sublayer=sublayer)
    assert L.moe.wait_failures() == 0


@pytest.mark.parametrize("D,I,G,E,k,shared,meta,router_dtype", [
    (256, 128, 32, 64, 6, False, osm_hip.F32, osm_hip.F32),
    (512, 256, 64, 100, 7, True, osm_hip.F16, osm_hip.BF16),
    (2048, 512, 128, 512, 11, True, osm_hip.BF16, osm_hip.BF16),
])
def test_single_launch_shapes(ctx, D, I, G, E, k, shared, meta, router_dtype):
    # Intermediate 128 / 256 / 512 (4, 8, 16 lanes per down row), f32 / f16 /
    # bf16 metadata, f32 and bf16 routers, with and without the shared
    # expert, top_k + shared up to the 12 slots the single launch takes.
    rng = np.random.default_rng(D + I + E + k)
    ometa = {osm_hip.F32: O.META_F32, osm_hip.F16: O.META_F16, osm_hip.BF16: O.META_BF16}[meta]
    g = osm_hip.geometry(D, I, G, meta)
    blobs = [random_blob(rng, D, I, G, ometa)[0] for _ in range(E)]
    slab = osm_hip.ExpertSlab(ctx, g, 1, E)
    for e in range(E):
        slab.upload(0, e, blobs[e])
    # Logits of order 1, as with the reference's N(0, 0.02) router at hidden
    # 2048, where the 1e-6 weight bar applies.
    router_f = rng.normal(0, 0.9 / np.sqrt(D), (E, D)).astype(np.float32)
    sg_f = rng.normal(0, 0.02, D).astype(np.float32)
    if router_dtype == osm_hip.BF16:
        router, sg = bf16_bits(router_f), bf16_bits(sg_f)
        router_f, sg_f = O.bf16_bits_to_f32(router), O.bf16_bits_to_f32(sg)
    else:
        router, sg = router_f, sg_f
    shared_blob = random_blob(rng, D, I, G, ometa)[0] if shared else None
    moe = osm_hip.MoeLayer(ctx, g, E, k, router, router_dtype, sg if shared else None, None, shared_blob,
                           max_tokens=1)
    for t in range(3):
        x = rng.normal(0, 1, (1, D)).astype(np.float32)
        one, three = both_paths(moe, slab, x)
        assert_same_bits(one, three)
        ora = O.qwen_sparse_moe(x[0], router_f, blobs, shared_blob, sg_f if shared else None, D, I, G, ometa, k)
        assert np.array_equal(one["ids"][0], ora["ids"])
        assert max_abs(one["weights"][0], ora["weights"]) <= 1e-6
        assert rel_l2(one["out"][0], ora["out"]) <= 1e-3
    assert moe.wait_failures() == 0


def test_single_launch_many_launches_device_resident(ctx):
    # Forty launches of one layer in a row, device pointers in and out (the
    # counters advance every launch and are never reset), each checked against
    # the per-token kernels on the same input.
    seed = 63
    L = QwenLayer(ctx, seed, max_tokens=1)
    n = 40
    xs = O.synth_tokens(seed, 800, n, L.D)
    x_dev, y1, y3 = ctx.alloc(n * L.D * 4), ctx.alloc(n * L.D * 4), ctx.alloc(n * L.D * 4)
    x_dev.upload(xs)
    row = L.D * 4
    L.moe.set_path(osm_hip.PATH_SINGLE_LAUNCH)
    for t in range(n):
        L.moe.decode_device(L.slab, 0, x_dev.ptr.value + t * row, y1.ptr.value + t * row, 1)
    L.moe.set_path(osm_hip.PATH_PER_TOKEN)
    for t in range(n):
        L.moe.decode_device(L.slab, 0, x_dev.ptr.value + t * row, y3.ptr.value + t * row, 1)
    ctx.synchronize()
    a = y1.download(np.float32, n * L.D)
    b = y3.download(np.float32, n * L.D)
    assert np.array_equal(a, b)
    assert L.moe.wait_failures() == 0


def test_single_launch_rejected_for_unsupported_shape(ctx):
    # top_k + shared = 17 slots: the layer keeps the per-token kernels.
    g = osm_hip.geometry(256, 128, 64, osm_hip.F32)
    router = np.random.default_rng(1).normal(0, 0.1, (64, 256)).astype(np.float32)
    moe = osm_hip.MoeLayer(ctx, g, 64, 16, router, osm_hip.F32,
                           np.zeros(256, np.float32), None, np.zeros(O.expert_blob_bytes(256, 128, 64, O.META_F32), np.uint8),
                           max_tokens=1)
    with pytest.raises(osm_hip.OsmError):
        moe.set_path(osm_hip.PATH_SINGLE_LAUNCH)
    moe.set_path(osm_hip.PATH_AUTO)
