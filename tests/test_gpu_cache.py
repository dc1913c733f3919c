"""The HBM-resident expert cache on the device.

The reference's own scenario (tests/vulkan_resident_expert_cache_test.cpp:
316-382) with its fixture experts and tolerance, and the cached routed-MoE
decode (capped budget, misses filled from pinned host memory) against the
all-resident decode and the restated cache policy."""

import os

import numpy as np
import pytest

import oracle as O
import osm_hip
from helpers import (blob_to_slot, cache_fixture_expert, cache_fixture_token, correlated_trace, max_abs,
                     qpack_q4_sections, rel_l2, write_qpack)

pytestmark = pytest.mark.gpu


def test_resident_cache_reference_scenario(ctx):
    # Budget of two experts; E0, E1 miss; E0 hits without touching the host
    # cache; E2 misses and evicts E1 (frequency 1 < E0's 2).
    g = osm_hip.geometry(128, 64, 64, osm_hip.BF16)
    blobs = [cache_fixture_expert(e) for e in range(3)]
    stride = blobs[0].size

    def read(layers, experts, dests):
        for l, e, d in zip(layers, experts, dests):
            d[:] = blobs[e]
        return 0

    host = osm_hip.HostExpertCache(stride, stride, read, minimum_slots=1)
    cache = osm_hip.ExpertCache(ctx, 2 * stride, host_cache=host, g=g)
    cache.get(0, 0)
    cache.get(0, 1)
    st = cache.stats()
    assert (st["hits"], st["misses"], st["loads"], st["evictions"]) == (0, 2, 2, 0)
    assert st["resident_entries"] == 2 and st["resident_bytes"] == 2 * stride

    before = host.stats()
    cache.get(0, 0)
    after = host.stats()
    assert (after["hits"], after["misses"]) == (before["hits"], before["misses"])  # a GPU hit bypasses L1

    cache.get(0, 2)
    st = cache.stats()
    assert (st["hits"], st["misses"], st["loads"], st["evictions"]) == (1, 3, 3, 1)
    assert st["resident_entries"] == 2 and st["resident_bytes"] <= st["budget_bytes"]
    assert cache.contains(0, 0) and not cache.contains(0, 1) and cache.contains(0, 2)

    for e in (0, 2):
        x = cache_fixture_token(e)
        got = cache.run(0, e, x)
        assert max_abs(got, O.expert_forward(blobs[e], 128, 64, 64, O.META_BF16, x)) <= 0.01
    st = cache.stats()
    assert (st["hits"], st["misses"], st["loads"], st["evictions"]) == (3, 3, 3, 1)


def test_cached_decode_matches_resident_decode(ctx):
    # A capped cache (12 of 2 x 64 experts) filled from pinned host memory on
    # the side stream: every token's output and routing must be the bits of
    # the all-resident decode, and the hit/miss/eviction counts those of the
    # restated policy replayed over the same picks (routed_moe.cpp:320-404
    # fetches the picks in order).
    seed, D, I, G, E, k, layers = 21, 256, 128, 64, 64, 4, 2
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    store = osm_hip.ExpertStore(g, layers, E)
    store.synthesize(ctx, seed)
    slab = osm_hip.ExpertSlab(ctx, g, layers, E)
    slab.synthesize(seed)
    stride = store.stride
    cache = osm_hip.ExpertCache(ctx, 12 * stride, store=store)
    policy = O.DeviceCachePolicy(12 * stride)
    moes = [osm_hip.MoeLayer(ctx, g, E, k, O.synth_router_bf16(seed, l, E, D), osm_hip.BF16,
                             O.synth_shared_gate_bf16(seed, l, D), O.synth_norm_weight(seed, l, D),
                             O.synth_expert_blob(seed, l, O.SHARED_EXPERT_ID, D, I, G), max_tokens=1)
            for l in range(layers)]
    x = O.synth_tokens(seed, 0, 12, D)
    for t in range(12):
        l = t % layers
        sub = t % 3 == 0
        got = moes[l].run_cached(cache, l, x[t], sublayer=sub)
        ref = moes[l].run_slab(slab, l, x[t], sublayer=sub)
        assert np.array_equal(got["ids"], ref["ids"])
        assert np.array_equal(got["weights"], ref["weights"])
        assert np.array_equal(got["out"], ref["out"])
        for e in got["ids"][0]:
            policy.get(l, int(e), stride)
    st, po = cache.stats(), policy.stats()
    for key in ("hits", "misses", "loads", "evictions", "resident_entries", "resident_bytes"):
        assert st[key] == po[key], (key, st, po)
    assert po["evictions"] > 0  # the cap was exercised
    assert cache.bytes_filled == st["loads"] * stride


def test_cached_decode_with_given_picks(ctx):
    # Caller-chosen routed experts through the capped cache: the output is the
    # pick-weighted sum of the chosen experts plus the router's sigmoid gate
    # times the shared expert (the composition of routed_moe.cpp:320-404 with
    # the routing replaced); ids and weights come back as given.
    seed, D, I, G, E, k = 22, 256, 128, 64, 64, 4
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    store = osm_hip.ExpertStore(g, 1, E)
    store.synthesize(ctx, seed)
    stride = store.stride
    cache = osm_hip.ExpertCache(ctx, 6 * stride, store=store)
    sg_bits = O.synth_shared_gate_bf16(seed, 0, D)
    shared = O.synth_expert_blob(seed, 0, O.SHARED_EXPERT_ID, D, I, G)
    moe = osm_hip.MoeLayer(ctx, g, E, k, O.synth_router_bf16(seed, 0, E, D), osm_hip.BF16, sg_bits, None, shared,
                           max_tokens=1)
    rng = np.random.default_rng(seed)
    sg = O.bf16_bits_to_f32(sg_bits)
    for t in range(5):
        x = O.synth_tokens(seed, t, 1, D)
        ids = rng.choice(E, k, replace=False).astype(np.uint32).reshape(1, k)
        w = rng.random(k).astype(np.float32)
        w = (w / w.sum()).astype(np.float32).reshape(1, k)
        got = moe.run_cached(cache, 0, x, picks=(ids, w))
        assert np.array_equal(got["ids"], ids) and np.array_equal(got["weights"], w)
        gate = 1.0 / (1.0 + np.exp(-np.dot(sg.astype(np.float64), x[0].astype(np.float64))))
        assert abs(got["shared_gate"][0] - gate) <= 1e-6
        ref = np.zeros(D, np.float64)
        for j in range(k):
            ref += float(w[0, j]) * O.expert_forward(store.blob_view(0, int(ids[0, j])), D, I, G, O.META_BF16, x[0])
        ref += float(got["shared_gate"][0]) * O.expert_forward(shared, D, I, G, O.META_BF16, x[0])
        assert rel_l2(got["out"][0], ref.astype(np.float32)) <= 1e-3
    assert cache.stats()["evictions"] > 0  # 20 picks over a 6-expert budget
    bad = np.array([[0, 1, 2, E]], np.uint32)
    with pytest.raises(osm_hip.OsmError):
        moe.run_cached(cache, 0, x, picks=(bad, w))
    with pytest.raises(osm_hip.OsmError):
        moe.run_cached(cache, 0, x, picks=(ids, np.full((1, k), np.nan, np.float32)))


def test_cached_batch_refills_its_own_slot(ctx):
    # A 4-expert budget, experts 0-3 used twice each. Picks [4, 5, 0, 1]: 4
    # misses and takes 0's slot (oldest of equal frequency), 5 misses and
    # would evict 4 (frequency 1, this call's own fill), 0 misses and would
    # evict 5 (restated policy: 3 evictions). As the reference runs each pick
    # right after its get (routed_moe.cpp:320-366), the call runs in rounds
    # -- {4}, then {5} once 4's round has read the slot, then {0, 1} -- and
    # its output is the oracle's sum of all four. The slot then holds 0's
    # bytes, the last of its three copies: the later all-hit calls are
    # checked against the oracle too.
    seed, D, I, G, E, k = 23, 256, 128, 64, 16, 4
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    store = osm_hip.ExpertStore(g, 1, E)
    store.synthesize(ctx, seed)
    cache = osm_hip.ExpertCache(ctx, 4 * store.stride, store=store)
    moe = osm_hip.MoeLayer(ctx, g, E, k, O.synth_router_bf16(seed, 0, E, D), osm_hip.BF16, None, None, None,
                           max_tokens=1)
    w = np.full((1, k), 1.0 / k, np.float32)

    def check(ids, t):
        x = O.synth_tokens(seed, t, 1, D)
        got = moe.run_cached(cache, 0, x, picks=(np.array([ids], np.uint32), w))
        ref = np.zeros(D, np.float64)
        for e in ids:
            ref += float(w[0, 0]) * O.expert_forward(store.blob_view(0, e), D, I, G, O.META_BF16, x[0])
        assert rel_l2(got["out"][0], ref.astype(np.float32)) <= 1e-3, (ids, t)

    check([0, 1, 2, 3], 0)
    check([0, 1, 2, 3], 1)
    check([4, 5, 0, 1], 2)
    assert cache.stats()["evictions"] == 3
    check([0, 1, 2, 3], 3)
    check([1, 2, 3, 0], 4)
    assert cache.stats()["evictions"] == 3  # both were all hits


def test_cached_two_tokens_refill_an_earlier_pick(ctx):
    # Two tokens in one call over a 4-expert budget warmed with 10-13 at
    # frequency 2, picking [0, 1] and [1, 0]: 0 is copied into 10's slot,
    # 1 evicts 0 and is copied into that same slot, 1 hits, and 0 is
    # admitted again into 11's slot. Token 0's first pick must read 0's
    # bytes from its final slot, not 1's from the slot it was first copied
    # to. Both tokens against the oracle; counters against the restated
    # policy.
    seed, D, I, G, E, k = 26, 256, 128, 64, 16, 2
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    store = osm_hip.ExpertStore(g, 1, E)
    store.synthesize(ctx, seed)
    stride = store.stride
    cache = osm_hip.ExpertCache(ctx, 4 * stride, store=store)
    policy = O.DeviceCachePolicy(4 * stride)
    sg_bits = O.synth_shared_gate_bf16(seed, 0, D)
    shared = O.synth_expert_blob(seed, 0, O.SHARED_EXPERT_ID, D, I, G)
    moe = osm_hip.MoeLayer(ctx, g, E, k, O.synth_router_bf16(seed, 0, E, D), osm_hip.BF16, sg_bits, None, shared,
                           max_tokens=2)
    sg = O.bf16_bits_to_f32(sg_bits)

    def run(ids, t0):
        ids = np.array(ids, np.uint32)
        n = ids.shape[0]
        w = np.tile(np.array([0.625, 0.375], np.float32), (n, 1))
        x = O.synth_tokens(seed, t0, n, D)
        got = moe.run_cached(cache, 0, x.reshape(-1), picks=(ids, w))
        for t in range(n):
            for e in ids[t]:
                policy.get(0, int(e), stride)
            gate = float(got["shared_gate"][t])
            ref_gate = 1.0 / (1.0 + np.exp(-np.dot(sg.astype(np.float64), x[t].astype(np.float64))))
            assert abs(gate - ref_gate) <= 1e-6
            ref = np.zeros(D, np.float64)
            for j in range(k):
                ref += float(w[t, j]) * O.expert_forward(store.blob_view(0, int(ids[t, j])), D, I, G, O.META_BF16, x[t])
            ref += gate * O.expert_forward(shared, D, I, G, O.META_BF16, x[t])
            assert rel_l2(got["out"][t], ref.astype(np.float32)) <= 1e-3, (ids.tolist(), t)

    for t0 in range(2):
        run([[10, 11]], 2 * t0)
        run([[12, 13]], 2 * t0 + 1)
    run([[0, 1], [1, 0]], 10)
    st, po = cache.stats(), policy.stats()
    for key in ("hits", "misses", "loads", "evictions", "resident_entries"):
        assert st[key] == po[key], (key, st, po)
    assert cache.contains(0, 0) and cache.contains(0, 1) and not cache.contains(0, 10)


@pytest.mark.parametrize("pinned", [True, False], ids=["pinned-kernel-fill", "pageable-dma-fill"])
def test_cached_decode_from_pread_storage(ctx, tmp_path, pinned):
    # The whole miss path from files: pread storage -> host L1 cache -> HBM
    # cache, against the all-resident decode (bit-identical outputs). With
    # pinned L1 slots a miss is filled by a kernel that reads the host pages;
    # with pageable slots, by the DMA engine.
    seed, D, I, G, E, k = 24, 256, 128, 64, 32, 4
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    slab = osm_hip.ExpertSlab(ctx, g, 1, E)
    slab.synthesize(seed)
    stride = osm_hip.expert_blob_bytes(g)
    os.makedirs(tmp_path / "packed_experts")
    np.concatenate([O.synth_expert_blob(seed, 0, e, D, I, G) for e in range(E)]).tofile(
        osm_hip.PreadStorage.layer_path(str(tmp_path), 0))
    storage = osm_hip.PreadStorage(str(tmp_path), 1, E, stride)
    # 16 HBM slots: the restated policy replayed over these tokens' routing
    # evicts 13 times and never a pick of the batch being made resident (at
    # 12 slots the last two tokens would lose one; the layer needs all of a
    # token's picks resident at once).
    host = osm_hip.HostExpertCache.from_storage(storage, 20 * stride, pinned=pinned)
    cache = osm_hip.ExpertCache(ctx, 16 * stride, host_cache=host, g=g)
    moe = osm_hip.MoeLayer(ctx, g, E, k, O.synth_router_bf16(seed, 0, E, D), osm_hip.BF16,
                           O.synth_shared_gate_bf16(seed, 0, D), O.synth_norm_weight(seed, 0, D),
                           O.synth_expert_blob(seed, 0, O.SHARED_EXPERT_ID, D, I, G), max_tokens=1)
    x = O.synth_tokens(seed, 0, 12, D)
    for t in range(12):
        got = moe.run_cached(cache, 0, x[t], sublayer=t % 2 == 0)
        ref = moe.run_slab(slab, 0, x[t], sublayer=t % 2 == 0)
        assert np.array_equal(got["ids"], ref["ids"]) and np.array_equal(got["out"], ref["out"])
    assert cache.stats()["evictions"] > 0 and host.stats()["misses"] > 0


def test_cached_decode_from_noncanonical_qpack(ctx, tmp_path):
    # A qpack container whose slots hold the nine sections in another order,
    # spaced apart, after an unrelated section: layout.json parsed and
    # checked, each slot read by pread and repacked into the blob, filled
    # from pinned host memory into 16 HBM slots, then decoded. Layer 1 of a
    # two-layer container is the one decoded. Outputs match the all-resident
    # decode bit for bit, and the oracle's routing and output.
    seed, D, I, G, E, k = 25, 256, 128, 64, 32, 4
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    order = ["up_proj.scales", "down_proj.weight", "gate_proj.biases", "up_proj.weight", "gate_proj.weight",
             "down_proj.biases", "up_proj.biases", "down_proj.scales", "gate_proj.scales"]
    secs, stride = qpack_q4_sections(D, I, G, "BF16", order=order, gap=40, extra=[("lm_hint", "F32", (9,), 36)])
    blobs = [[O.synth_expert_blob(seed, l, e, D, I, G) for e in range(E)] for l in range(2)]
    write_qpack(str(tmp_path), [np.stack([blob_to_slot(b, secs, stride, D, I, G, "BF16") for b in layer])
                                for layer in blobs], secs, stride, linear_layers=[True, False], quant_group_size=G)
    storage = osm_hip.QpackStorage(str(tmp_path), g)
    assert storage.stride == osm_hip.expert_blob_bytes(g) < stride
    host = osm_hip.HostExpertCache.from_storage(storage, 20 * storage.stride, pinned=True)
    cache = osm_hip.ExpertCache(ctx, 16 * storage.stride, host_cache=host, g=g)
    slab = osm_hip.ExpertSlab(ctx, g, 1, E)
    for e in range(E):
        slab.upload(0, e, blobs[1][e])
    router = O.synth_router_bf16(seed, 1, E, D)
    sg = O.synth_shared_gate_bf16(seed, 1, D)
    norm = O.synth_norm_weight(seed, 1, D)
    shared = O.synth_expert_blob(seed, 1, O.SHARED_EXPERT_ID, D, I, G)
    moe = osm_hip.MoeLayer(ctx, g, E, k, router, osm_hip.BF16, sg, norm, shared, max_tokens=1)
    rf, sgf = O.bf16_bits_to_f32(router), O.bf16_bits_to_f32(sg)
    x = O.synth_tokens(seed, 1, 12, D)
    for t in range(12):
        sub = t % 2 == 0
        got = moe.run_cached(cache, 1, x[t], sublayer=sub)
        ref = moe.run_slab(slab, 0, x[t], sublayer=sub)
        assert np.array_equal(got["ids"], ref["ids"]) and np.array_equal(got["out"], ref["out"]), t
        if sub:
            ora = O.moe_sublayer(x[t], norm, 1e-6, rf, blobs[1], shared, sgf, D, I, G, O.META_BF16, k)
        else:
            ora = O.qwen_sparse_moe(x[t], rf, blobs[1], shared, sgf, D, I, G, O.META_BF16, k)
        assert np.array_equal(np.asarray(got["ids"]).reshape(-1), ora["ids"]), t
        assert rel_l2(np.asarray(got["out"]).reshape(-1), ora["out"]) <= 1e-3, t
    assert cache.stats()["evictions"] > 0 and host.stats()["misses"] > 0


def test_cached_layer_stack_matches_layer_calls(ctx):
    # The native stack of cached sublayers against one call per layer: the
    # same outputs bit for bit, with given picks and with device routing.
    seed, D, I, G, E, k, layers = 25, 256, 128, 64, 32, 4, 3
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    store = osm_hip.ExpertStore(g, layers, E)
    store.synthesize(ctx, seed)
    moes = [osm_hip.MoeLayer(ctx, g, E, k, O.synth_router_bf16(seed, l, E, D), osm_hip.BF16,
                             O.synth_shared_gate_bf16(seed, l, D), O.synth_norm_weight(seed, l, D),
                             O.synth_expert_blob(seed, l, O.SHARED_EXPERT_ID, D, I, G), max_tokens=1)
            for l in range(layers)]
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(layers)]).astype(np.uint32).reshape(layers, 1, k)
    w = rng.random((layers, 1, k)).astype(np.float32)
    x = O.synth_tokens(seed, 0, 1, D)
    for picks in ((ids, w), None):
        a = osm_hip.ExpertCache(ctx, 64 * store.stride, store=store)
        b = osm_hip.ExpertCache(ctx, 64 * store.stride, store=store)
        got = osm_hip.run_cached_layers(ctx, moes, list(range(layers)), a, x, picks)
        ref = x
        for l in range(layers):
            p = (ids[l], w[l]) if picks is not None else None
            ref = moes[l].run_cached(b, l, ref, sublayer=True, picks=p)["out"]
        assert np.array_equal(got, ref)
        assert a.stats()["misses"] == b.stats()["misses"] > 0


class SmallStack:
    """Four sublayers of top-4 over 32 experts (hidden 256): a pinned host copy
    of every expert, an all-resident slab of the same weights, the layers."""

    seed, D, I, G, E, k, L = 31, 256, 128, 64, 32, 4, 4

    def __init__(self, ctx):
        s = self
        s.g = osm_hip.geometry(s.D, s.I, s.G, osm_hip.BF16)
        s.store = osm_hip.ExpertStore(s.g, s.L, s.E)
        s.store.synthesize(ctx, s.seed)
        s.slab = osm_hip.ExpertSlab(ctx, s.g, s.L, s.E)
        s.slab.synthesize(s.seed)
        s.norm = [O.synth_norm_weight(s.seed, l, s.D) for l in range(s.L)]
        s.sg = [O.synth_shared_gate_bf16(s.seed, l, s.D) for l in range(s.L)]
        s.shared = [O.synth_expert_blob(s.seed, l, O.SHARED_EXPERT_ID, s.D, s.I, s.G) for l in range(s.L)]
        s.moes = [osm_hip.MoeLayer(ctx, s.g, s.E, s.k, O.synth_router_bf16(s.seed, l, s.E, s.D), osm_hip.BF16,
                                   s.sg[l], s.norm[l], s.shared[l], max_tokens=2) for l in range(s.L)]

    def oracle_chain(self, x, ids, w):
        """The given-picks sublayers chained on the oracle."""
        s = self
        for l in range(s.L):
            blobs = [O.synth_expert_blob(s.seed, l, int(e), s.D, s.I, s.G) for e in ids[l][0]]
            x = O.moe_sublayer_picks(x, s.norm[l], 1e-6, w[l][0], blobs, s.shared[l], O.bf16_bits_to_f32(s.sg[l]),
                                     s.D, s.I, s.G, O.META_BF16)
        return x


@pytest.mark.parametrize("slots", [64, 6, 3, 1])
def test_cached_stack_under_eviction_given_picks(ctx, slots):
    # The capped-cache stack with given picks (the 48-layer bench's path) on
    # a correlated trace (p = 0.6), with a budget of 64 experts (all fit),
    # 6 (about 1.5 k: a slot is refilled within one or two layers), 3 and 1
    # (below k: a layer's picks run in rounds, each ending just before a get
    # would evict one of its picks, routed_moe.cpp:320-366):
    #  - the stack in one native call equals the layer-by-layer calls on a
    #    second cache, bit for bit, token after token;
    #  - every budget gives the bits of the 64-expert budget (the fused
    #    kernels), so the rounds' partials and their combine change nothing;
    #  - both caches' counters equal the restated policy over the picks;
    #  - two tokens' outputs are within 1e-3 of the oracle's chain.
    S = SmallStack(ctx)
    steps = 8
    rng = np.random.default_rng(5)
    trace = correlated_trace(rng, S.L, steps, S.k, S.E, 0.6)
    w = rng.random((steps, S.L, 1, S.k)).astype(np.float32)
    w /= w.sum(axis=-1, keepdims=True)
    xs = O.synth_tokens(S.seed, 40, steps, S.D)
    stride = S.store.stride

    def run(budget):
        a = osm_hip.ExpertCache(ctx, budget * stride, store=S.store)
        b = osm_hip.ExpertCache(ctx, budget * stride, store=S.store)
        policy = O.DeviceCachePolicy(budget * stride)
        outs = []
        for s in range(steps):
            ids = np.stack(trace[s])
            got = osm_hip.run_cached_layers(ctx, S.moes, list(range(S.L)), a, xs[s], (ids, w[s]))
            ref = xs[s]
            for l in range(S.L):
                ref = S.moes[l].run_cached(b, l, ref, sublayer=True, picks=(ids[l], w[s][l]))["out"]
                for e in ids[l][0]:
                    policy.get(l, int(e), stride)
            assert np.array_equal(got.reshape(-1), np.asarray(ref).reshape(-1)), (budget, s)
            outs.append(got.reshape(-1))
        st, sb, po = a.stats(), b.stats(), policy.stats()
        for key in ("hits", "misses", "loads", "evictions", "resident_entries"):
            assert st[key] == sb[key] == po[key], (budget, key, st, sb, po)
        a.close()
        b.close()
        return outs, st

    outs, st = run(slots)
    if slots < 64:
        assert st["evictions"] > 0, st
        full, _ = run(64)
        for s in range(steps):
            assert np.array_equal(outs[s], full[s]), (slots, s)
    for s in (0, steps - 1):
        ids = np.stack(trace[s])
        assert rel_l2(outs[s], S.oracle_chain(xs[s], ids, w[s])) <= 1e-3, (slots, s)


@pytest.mark.parametrize("slots", [6, 3, 1])
def test_cached_stack_under_eviction_device_routing(ctx, slots):
    # The same stack routed on the device: each layer's ids come back to the
    # host, the picks already resident run while the misses are copied, and
    # below k a layer's picks run in rounds. The stack in one call, the
    # layer-by-layer calls on a second cache and the all-resident slab decode
    # give the same bits; the counters equal the restated policy over the
    # slab decode's routing.
    S = SmallStack(ctx)
    steps = 8
    xs = O.synth_tokens(S.seed, 70, steps, S.D)
    stride = S.store.stride
    a = osm_hip.ExpertCache(ctx, slots * stride, store=S.store)
    b = osm_hip.ExpertCache(ctx, slots * stride, store=S.store)
    policy = O.DeviceCachePolicy(slots * stride)
    for s in range(steps):
        got = osm_hip.run_cached_layers(ctx, S.moes, list(range(S.L)), a, xs[s])
        ref = res = xs[s]
        for l in range(S.L):
            ref = S.moes[l].run_cached(b, l, ref, sublayer=True)["out"]
            r = S.moes[l].run_slab(S.slab, l, res, sublayer=True)
            res = r["out"]
            for e in r["ids"][0]:
                policy.get(l, int(e), stride)
        assert np.array_equal(got.reshape(-1), np.asarray(ref).reshape(-1)), (slots, s)
        assert np.array_equal(got.reshape(-1), np.asarray(res).reshape(-1)), (slots, s)
    st, sb, po = a.stats(), b.stats(), policy.stats()
    for key in ("hits", "misses", "loads", "evictions", "resident_entries"):
        assert st[key] == sb[key] == po[key], (slots, key, st, sb, po)
    assert st["evictions"] > 0, st
