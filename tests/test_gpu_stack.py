"""The 48-layer Qwen3-Next-80B-A3B-shaped stack of MoE sublayers, one token
per decode step, as the reference's decoder stack runs its layers in order
(src/model/checkpoint_decoder_stack.cpp:191-204, each layer a
QwenCheckpointMoeSublayer::run, src/model/checkpoint_moe_sublayer.cpp:138-199).

512 experts plus a shared expert per layer, 43.5 GB of q4 experts:
(a) every expert resident in HBM: every layer of two decode steps against the
    oracle's sublayer on the same input (ids bit-exact, the MoE part of the
    output within 1e-3 relative L2), and the whole chain against a chain of
    the oracle's sublayers (ids bit-exact at every layer, final output within
    1e-3 relative L2);
(b) the HBM cache capped at 16 GB, misses filled from a pinned host copy of
    the 43.5 GB: decode steps until the cache has evicted for 16 steps,
    bit-identical to the resident stack, with
    the cache counters equal to the restated LFU+recency policy replayed over
    the resident stack's routing;
(c) the same capped cache driven by a correlated routing trace (each of a
    layer's 10 picks repeats one of its previous-step picks with p = 0.6,
    the benchmark's workload) through the pipelined stack: bit-identical to
    the layer-by-layer calls on a second cache until both have evicted for
    16 steps, counters equal to the restated policy, and two tokens within
    1e-3 of the oracle's chain of given-picks sublayers.
"""

import numpy as np
import pytest

import oracle as O
import osm_hip
from helpers import correlated_trace, pmap, rel_l2

pytestmark = pytest.mark.gpu

LAYERS, D, I, G, E, K = 48, 2048, 512, 64, 512, 10
SEED = 2024
CACHE_BYTES = 16 * 10**9


class Stack:
    def __init__(self, ctx):
        self.ctx = ctx
        self.g = osm_hip.geometry(D, I, G, osm_hip.BF16)
        self.slab = osm_hip.ExpertSlab(ctx, self.g, LAYERS, E)
        self.slab.synthesize(SEED)
        self.router = [O.synth_router_bf16(SEED, l, E, D) for l in range(LAYERS)]
        self.sg = [O.synth_shared_gate_bf16(SEED, l, D) for l in range(LAYERS)]
        self.norm = [O.synth_norm_weight(SEED, l, D) for l in range(LAYERS)]
        self.shared = [O.synth_expert_blob(SEED, l, O.SHARED_EXPERT_ID, D, I, G) for l in range(LAYERS)]
        self.layers = [osm_hip.MoeLayer(ctx, self.g, E, K, self.router[l], osm_hip.BF16, self.sg[l], self.norm[l],
                                        self.shared[l], max_tokens=1) for l in range(LAYERS)]
        self.x, self.y, self.scratch = (ctx.alloc(D * 4) for _ in range(3))

    def step(self, x):
        """One decode step through all layers in one native call: final y."""
        self.x.upload(np.ascontiguousarray(x, np.float32))
        osm_hip.decode_layers(self.ctx, self.layers, list(range(LAYERS)), self.slab, self.x.ptr, self.y.ptr,
                              self.scratch.ptr, 1, True)
        return self.y.download(np.float32, D)

    def step_by_layer(self, x):
        """The same step one layer call at a time: every layer's input, and
        its routing read back from the layer."""
        xs, ids = [np.ascontiguousarray(x, np.float32)], []
        for l in range(LAYERS):
            self.x.upload(xs[-1])
            osm_hip.decode_layers(self.ctx, [self.layers[l]], [l], self.slab, self.x.ptr, self.y.ptr,
                                  self.scratch.ptr, 1, True)
            xs.append(self.y.download(np.float32, D))
            ids.append(self.layers[l].routing(1)["ids"][0])
        return xs, ids

    def oracle_layer(self, l, x, blobs):
        router = O.bf16_bits_to_f32(self.router[l])
        xin = O.rms_norm(x, 1, D, self.norm[l], 1e-6)
        picks = O.route_qwen_top_k(xin, router, D, E, K, True)
        for e in picks["ids"]:
            if (l, int(e)) not in blobs:
                blobs[(l, int(e))] = O.synth_expert_blob(SEED, l, int(e), D, I, G)
        dummy = blobs[(l, int(picks["ids"][0]))]
        table = [blobs.get((l, e), dummy) for e in range(E)]
        r = O.moe_sublayer(x, self.norm[l], 1e-6, router, table, self.shared[l], O.bf16_bits_to_f32(self.sg[l]),
                           D, I, G, O.META_BF16, K)
        assert np.array_equal(r["ids"], picks["ids"])
        return r


@pytest.fixture(scope="module")
def stack(ctx):
    s = Stack(ctx)
    yield s
    for m in s.layers:
        m.close()
    s.slab.close()


def test_resident_stack_against_oracle(stack):
    tokens = O.synth_tokens(SEED, 0, 2, D)
    for t in range(2):
        y = stack.step(tokens[t])
        xs, ids = stack.step_by_layer(tokens[t])
        assert np.array_equal(xs[-1], y)  # one native call == layer by layer, bit for bit
        # Every layer against the oracle's sublayer on the same input.
        blobs = {}

        def check(l):
            r = stack.oracle_layer(l, xs[l], blobs)
            return r["ids"], rel_l2((xs[l + 1].astype(np.float64) - xs[l]), (r["out"].astype(np.float64) - xs[l]))

        for l, (ora_ids, err) in enumerate(pmap(check, range(LAYERS))):
            assert np.array_equal(ids[l], ora_ids), (t, l, list(ids[l]), list(ora_ids))
            assert err <= 1e-3, (t, l, err)
        # The whole chain against a chain of the oracle's sublayers.
        x = tokens[t].copy()
        for l in range(LAYERS):
            r = stack.oracle_layer(l, x, blobs)
            assert np.array_equal(ids[l], r["ids"]), (t, l, list(ids[l]), list(r["ids"]))
            x = r["out"]
        assert rel_l2(y, x) <= 1e-3, t


def test_capped_cache_stack_matches_resident(ctx, stack):
    store = osm_hip.ExpertStore(stack.g, LAYERS, E)
    store.synthesize(ctx, SEED)
    cache = osm_hip.ExpertCache(ctx, CACHE_BYTES, store=store)
    policy = O.DeviceCachePolicy(CACHE_BYTES)
    stride = store.stride
    # Routed by the device on fresh tokens, 64 steps touch about 8,500
    # distinct experts, fewer than the 9,042 slots of 16 GB: run until the
    # cache has evicted for 16 steps (at most 400 steps).
    t, evicting = 0, 0
    while evicting < 16:
        assert t < 400, cache.stats()
        x = O.synth_tokens(SEED, t, 1, D)[0]
        ref = stack.step(x)
        got = osm_hip.run_cached_layers(ctx, stack.layers, list(range(LAYERS)), cache, x)
        assert np.array_equal(got.reshape(D), ref), t
        for l in range(LAYERS):
            for e in stack.layers[l].routing(1)["ids"][0]:
                policy.get(l, int(e), stride)
        evicting += 1 if cache.stats()["evictions"] > 0 else 0
        t += 1
    st, po = cache.stats(), policy.stats()
    for key in ("hits", "misses", "loads", "evictions", "resident_entries"):
        assert st[key] == po[key], (key, st, po)
    assert st["evictions"] > 0 and st["resident_bytes"] <= CACHE_BYTES, st
    cache.close()
    store.close()


def test_capped_cache_given_trace_matches_layer_calls(ctx, stack):
    store = osm_hip.ExpertStore(stack.g, LAYERS, E)
    store.synthesize(ctx, SEED)
    a = osm_hip.ExpertCache(ctx, CACHE_BYTES, store=store)
    b = osm_hip.ExpertCache(ctx, CACHE_BYTES, store=store)
    policy = O.DeviceCachePolicy(CACHE_BYTES)
    stride = store.stride
    rng = np.random.default_rng(SEED + 7)
    steps = 120
    trace = correlated_trace(rng, LAYERS, steps, K, E, 0.6)
    w = np.arange(K, 0, -1, dtype=np.float32)
    w = np.broadcast_to((w / w.sum()).astype(np.float32).reshape(1, 1, K), (LAYERS, 1, K)).copy()
    xs = O.synth_tokens(SEED, 900000, steps, D)
    evicting, first_evicting, s = 0, None, 0
    checked = []
    while evicting < 16:
        assert s < steps, a.stats()
        ids = np.stack(trace[s])
        got = osm_hip.run_cached_layers(ctx, stack.layers, list(range(LAYERS)), a, xs[s], (ids, w))
        ref = xs[s]
        for l in range(LAYERS):
            ref = stack.layers[l].run_cached(b, l, ref, sublayer=True, picks=(ids[l], w[l]))["out"]
            for e in ids[l][0]:
                policy.get(l, int(e), stride)
        assert np.array_equal(got.reshape(D), np.asarray(ref).reshape(D)), s
        if a.stats()["evictions"] > 0:
            evicting += 1
            if first_evicting is None:
                first_evicting = s
        if s == 0 or evicting == 1:
            checked.append((s, got.reshape(D).copy()))
        s += 1
    st, sb, po = a.stats(), b.stats(), policy.stats()
    for key in ("hits", "misses", "loads", "evictions", "resident_entries"):
        assert st[key] == sb[key] == po[key], (key, st, sb, po)
    assert st["evictions"] > 0 and st["resident_bytes"] <= CACHE_BYTES, st
    # Two tokens (the first, and the first step that evicted) against the
    # oracle's chain of given-picks sublayers.
    for s, y in checked[:2]:
        ids = np.stack(trace[s])
        x = xs[s].copy()
        for l in range(LAYERS):
            picked = pmap(lambda e: O.synth_expert_blob(SEED, l, int(e), D, I, G), list(ids[l][0]))
            x = O.moe_sublayer_picks(x, stack.norm[l], 1e-6, w[l][0], picked, stack.shared[l],
                                     O.bf16_bits_to_f32(stack.sg[l]), D, I, G, O.META_BF16)
        assert rel_l2(y, x) <= 1e-3, s
    a.close()
    b.close()
    store.close()
