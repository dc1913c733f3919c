"""Resident experts and the routed-MoE layer on the device against the oracle.

Bars: routed expert ids bit-exact (order included: descending probability,
ties to the lower id); routing weights and the shared gate within 1e-6
absolute (tests/checkpoint_moe_sublayer_test.cpp:690-699); outputs within
1e-3 relative L2 of the fp32 CPU oracle, and within the reference's absolute
tolerances on its own small fixtures."""

import numpy as np
import pytest

import oracle as O
import osm_hip
from helpers import cache_fixture_expert, cache_fixture_token, max_abs, pmap, random_blob, rel_l2

pytestmark = pytest.mark.gpu

QWEN = dict(hidden=2048, inter=512, group=64, experts=512, top_k=10)


def test_synth_device_matches_host(ctx):
    g = osm_hip.geometry(2048, 512, 64, osm_hip.BF16)
    for layer, expert in [(0, 0), (3, 511), (47, 0xFFFFFFFF)]:
        assert np.array_equal(osm_hip.synth_expert_blob(ctx, 9, layer, expert, g), O.synth_expert_blob(9, layer, expert, 2048, 512))
    g32 = osm_hip.geometry(256, 64, 32, osm_hip.F32)
    assert np.array_equal(osm_hip.synth_expert_blob(ctx, 2, 1, 5, g32), O.synth_expert_blob(2, 1, 5, 256, 64, 32, O.META_F32))
    assert np.array_equal(osm_hip.synth_router_bf16(ctx, 9, 4, 512, 2048), O.synth_router_bf16(9, 4, 512, 2048))
    assert np.array_equal(osm_hip.synth_shared_gate_bf16(ctx, 9, 4, 2048), O.synth_shared_gate_bf16(9, 4, 2048))
    assert np.array_equal(osm_hip.synth_norm_weight(ctx, 9, 4, 2048).view(np.uint32), O.synth_norm_weight(9, 4, 2048).view(np.uint32))
    assert np.array_equal(osm_hip.synth_tokens(ctx, 9, 100, 5, 2048).view(np.uint32), O.synth_tokens(9, 100, 5, 2048).view(np.uint32))


# ---- single experts --------------------------------------------------------------------
def test_resident_expert_reference_fixture(ctx):
    # The 128 -> 64 -> 128 experts of tests/vulkan_resident_expert_cache_test.cpp (tolerance 0.01).
    g = osm_hip.geometry(128, 64, 64, osm_hip.BF16)
    for e in range(3):
        blob = cache_fixture_expert(e)
        ex = osm_hip.ResidentExpert(ctx, blob, g)
        assert ex.accounted_bytes == blob.size
        x = cache_fixture_token(e)
        gpu = ex.run(x)
        ora = O.expert_forward(blob, 128, 64, 64, O.META_BF16, x)
        assert max_abs(gpu, ora) <= 0.01 and rel_l2(gpu, ora) <= 1e-3


@pytest.mark.parametrize("meta", [osm_hip.BF16, osm_hip.F32, osm_hip.F16])
def test_resident_expert_qwen_shape(ctx, meta):
    # One expert, one token at the Qwen3-Next shape (2048 -> 512 -> 2048).
    g = osm_hip.geometry(2048, 512, 64, meta)
    rng = np.random.default_rng(20 + meta)
    blob, _ = random_blob(rng, 2048, 512, 64, meta)
    x = rng.normal(0, 1, 2048).astype(np.float32)
    ex = osm_hip.ResidentExpert(ctx, blob, g)
    gpu = ex.run(x)
    ora = O.expert_forward(blob, 2048, 512, 64, meta, x)
    assert rel_l2(gpu, ora) <= 1e-3
    xb = osm_hip.FloatBuffer(ctx, 2048)
    xb.upload(x)
    ex.run_from_buffer(xb)
    assert np.array_equal(ex.output(), gpu)


def test_resident_expert_rejects_bad_geometry(ctx):
    with pytest.raises(osm_hip.OsmError):
        osm_hip.ResidentExpert(ctx, np.zeros(100, np.uint8), osm_hip.geometry(100, 64, 64, osm_hip.BF16))
    with pytest.raises(osm_hip.OsmError):
        osm_hip.ResidentExpert(ctx, np.zeros(100, np.uint8), osm_hip.geometry(128, 64, 64, osm_hip.BF16))


def test_shared_expert(ctx):
    seed = 31
    g = osm_hip.geometry(2048, 512, 64, osm_hip.BF16)
    blob = O.synth_expert_blob(seed, 0, O.SHARED_EXPERT_ID, 2048, 512)
    sg = O.bf16_bits_to_f32(O.synth_shared_gate_bf16(seed, 0, 2048))
    x = O.synth_tokens(seed, 0, 1, 2048)[0]
    se = osm_hip.SharedExpert(ctx, blob, g, sg)
    logit = np.float32(0)
    for i in range(2048):
        logit = np.float32(logit + np.float32(sg[i] * x[i]))
    assert se.scalar_scale(x) == O.sigmoid(float(logit))
    xb = osm_hip.FloatBuffer(ctx, 2048)
    xb.upload(x)
    se.run_from_buffer(xb)
    assert rel_l2(se.output(), O.expert_forward(blob, 2048, 512, 64, O.META_BF16, x)) <= 1e-3


# ---- MoE layer ---------------------------------------------------------------------------
class QwenLayer:
    """One synthetic Qwen3-Next-shaped MoE layer: device slab + layer state, and
    the oracle's view of the same weights (experts regenerated on the host)."""

    def __init__(self, ctx, seed, layer=0, max_tokens=16, norm=False, **shape):
        sh = dict(QWEN, **shape)
        self.seed, self.layer = seed, layer
        self.D, self.I, self.G, self.E, self.k = sh["hidden"], sh["inter"], sh["group"], sh["experts"], sh["top_k"]
        self.g = osm_hip.geometry(self.D, self.I, self.G, osm_hip.BF16)
        self.slab = osm_hip.ExpertSlab(ctx, self.g, 1, self.E)
        self._synth_slab()
        self.router_bits = O.synth_router_bf16(seed, layer, self.E, self.D)
        self.sg_bits = O.synth_shared_gate_bf16(seed, layer, self.D)
        self.norm_w = O.synth_norm_weight(seed, layer, self.D) if norm else None
        self.shared = O.synth_expert_blob(seed, layer, O.SHARED_EXPERT_ID, self.D, self.I, self.G)
        self.moe = osm_hip.MoeLayer(ctx, self.g, self.E, self.k, self.router_bits, osm_hip.BF16, self.sg_bits,
                                    self.norm_w, self.shared, max_tokens=max_tokens)
        self._blobs = {}

    def _synth_slab(self):
        # The slab holds layer `self.layer` of the seeded model at slab layer 0.
        if self.layer == 0:
            self.slab.synthesize(self.seed)
        else:
            for e in range(self.E):
                self.slab.upload(0, e, O.synth_expert_blob(self.seed, self.layer, e, self.D, self.I, self.G))

    def blob(self, e):
        if e not in self._blobs:
            self._blobs[e] = O.synth_expert_blob(self.seed, self.layer, e, self.D, self.I, self.G)
        return self._blobs[e]

    def oracle_token(self, x, sublayer=False):
        router = O.bf16_bits_to_f32(self.router_bits)
        sg = O.bf16_bits_to_f32(self.sg_bits)
        xin = O.rms_norm(x, 1, self.D, self.norm_w, 1e-6) if sublayer else x
        picks = O.route_qwen_top_k(xin, router, self.D, self.E, self.k, True)
        dummy = self.blob(int(picks["ids"][0]))
        table = [self.blob(e) if e in set(int(i) for i in picks["ids"]) else dummy for e in range(self.E)]
        if sublayer:
            r = O.moe_sublayer(x, self.norm_w, 1e-6, router, table, self.shared, sg, self.D, self.I, self.G, O.META_BF16, self.k)
        else:
            r = O.qwen_sparse_moe(x, router, table, self.shared, sg, self.D, self.I, self.G, O.META_BF16, self.k)
        r["logits"] = picks["logits"]
        r["mass"] = picks["mass"]
        return r


def assert_weights(w_gpu, logits_gpu, ids, w_ora, logits_ora):
    """Routing weights: the reference's selection arithmetic applied to the
    device's own logits gives them within 1e-6 (reference_ops.cpp:130-212,
    qwen_router.cpp:72-91); against the oracle they may differ further only
    by what the logits' rounding explains. A weight is
    exp(l_i - m) / sum_sel exp(l_j - m), so a logit error d moves it by at
    most 2 * w * max|d| over the selected experts (at the Qwen3-Next shape
    the sequential fp32 sum of the reference and the device's tree sum
    differ by about 1e-6 in a logit)."""
    ids_own, w_own = O.route_top_k(logits_gpu, len(ids), True)
    assert np.array_equal(ids_own, ids)
    assert max_abs(w_gpu, w_own) <= 1e-6
    d = max_abs(logits_gpu[ids], logits_ora[ids])
    assert max_abs(w_gpu, w_ora) <= 1e-6 + 2.0 * float(np.max(w_ora)) * d, (max_abs(w_gpu, w_ora), d)


def assert_token_parity(gpu, t, ora, sublayer=False):
    ids_g, ids_o = gpu["ids"][t], ora["ids"]
    if not np.array_equal(ids_g, ids_o):
        lg = np.sort(ora["logits"])[::-1]
        pytest.fail(f"routed ids differ: gpu {list(ids_g)} oracle {list(ids_o)}; "
                    f"oracle logit gap k/k+1 = {lg[len(ids_o) - 1] - lg[len(ids_o)]:.3e}")
    assert_weights(gpu["weights"][t], gpu["logits"][t], ids_g, ora["weights"], ora["logits"])
    assert abs(gpu["shared_gate"][t] - ora["shared_gate"]) <= 1e-6
    assert rel_l2(gpu["logits"][t], ora["logits"]) <= 1e-5
    assert rel_l2(gpu["out"][t], ora["out"]) <= 1e-3
    if sublayer:
        assert max_abs(gpu["normalized"][t], ora["normalized"]) <= 1e-5


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_moe_decode_qwen_b1(ctx, seed):
    # One routed-MoE sublayer decode, batch 1: top-10 of 512 + gated shared expert.
    L = QwenLayer(ctx, seed)
    x = O.synth_tokens(seed, 0, 1, L.D)
    gpu = L.moe.run_slab(L.slab, 0, x)
    assert_token_parity(gpu, 0, L.oracle_token(x[0]))


def test_moe_sublayer_rmsnorm_residual(ctx):
    seed = 4
    L = QwenLayer(ctx, seed, norm=True)
    x = O.synth_tokens(seed, 0, 1, L.D) * np.float32(2.5)
    gpu = L.moe.run_slab(L.slab, 0, x, sublayer=True)
    assert_token_parity(gpu, 0, L.oracle_token(x[0], sublayer=True), sublayer=True)


@pytest.mark.parametrize("tokens", [4, 16, 64])
def test_moe_decode_batched(ctx, tokens):
    # Decode batch sizes 4, 16 and 64 through the per-token kernels: each
    # token routed independently (oracle: per-token loop, as
    # src/session/greedy_token_session.cpp:170-192 runs prefill).
    seed = 5
    L = QwenLayer(ctx, seed, max_tokens=64)
    L.moe.set_path(osm_hip.PATH_PER_TOKEN)
    x = O.synth_tokens(seed, 1000, tokens, L.D)
    gpu = L.moe.run_slab(L.slab, 0, x)
    for e in {int(i) for i in gpu["ids"].ravel()}:
        L.blob(e)  # fill the host blob cache before the oracle threads read it
    oras = pmap(lambda t: L.oracle_token(x[t]), range(tokens))
    for t in range(tokens):
        assert_token_parity(gpu, t, oras[t], sublayer=False)


def test_moe_small_reference_shapes_f32_router(ctx):
    # The reference's routed-MoE fixture sizes: hidden 128, intermediate 64,
    # 3 experts, top-2 (tests/weighted_routed_moe_test.cpp); fp32 router and
    # fp32 metadata, no shared expert.
    rng = np.random.default_rng(6)
    D, I, E, k = 128, 64, 3, 2
    g = osm_hip.geometry(D, I, 64, osm_hip.F32)
    blobs = [random_blob(rng, D, I, 64, O.META_F32)[0] for _ in range(E)]
    slab = osm_hip.ExpertSlab(ctx, g, 1, E)
    for e in range(E):
        slab.upload(0, e, blobs[e])
    router = rng.normal(0, 0.3, (E, D)).astype(np.float32)
    moe = osm_hip.MoeLayer(ctx, g, E, k, router, osm_hip.F32, max_tokens=2)
    x = rng.normal(0, 1, (2, D)).astype(np.float32)
    gpu = moe.run_slab(slab, 0, x)
    for t in range(2):
        ora = O.qwen_sparse_moe(x[t], router, blobs, None, None, D, I, 64, O.META_F32, k)
        assert np.array_equal(gpu["ids"][t], ora["ids"])
        assert max_abs(gpu["weights"][t], ora["weights"]) <= 1e-6
        assert abs(gpu["weights"][t].sum() - 1) <= 1e-6
        assert max_abs(gpu["out"][t], ora["out"]) <= 0.02 and rel_l2(gpu["out"][t], ora["out"]) <= 1e-3


@pytest.mark.parametrize("E,k,mode", [(100, 7, "random"), (1024, 10, "random"), (200, 16, "ties"),
                                      (64, 1, "ties"), (700, 16, "underflow"), (33, 16, "underflow")])
def test_moe_routing_edges(ctx, E, k, mode):
    # Selection corners against the oracle's router (reference_ops.cpp:130-212):
    # expert counts that leave lanes partly or wholly empty, exact ties (three
    # distinct router rows, so equal logits and probabilities: lower id first),
    # and logits hundreds apart, where exp underflows to 0 for all but a few
    # experts and the remaining picks are the lowest ids with probability 0.
    rng = np.random.default_rng(E * 31 + k)
    D, I, G = 128, 64, 64
    g = osm_hip.geometry(D, I, G, osm_hip.F32)
    blob = random_blob(rng, D, I, G, O.META_F32)[0]  # one blob everywhere: routing is under test
    slab = osm_hip.ExpertSlab(ctx, g, 1, E)
    for e in range(E):
        slab.upload(0, e, blob)
    if mode == "ties":
        rows = rng.normal(0, 0.3, (3, D)).astype(np.float32)
        router = rows[rng.integers(0, 3, E)]
    elif mode == "underflow":
        router = rng.normal(0, 30.0, (E, D)).astype(np.float32)
    else:
        router = rng.normal(0, 0.3, (E, D)).astype(np.float32)
    moe = osm_hip.MoeLayer(ctx, g, E, k, router, osm_hip.F32, max_tokens=2)
    x = rng.normal(0, 1, (2, D)).astype(np.float32)
    gpu = moe.run_slab(slab, 0, x)
    for t in range(2):
        ora = O.route_qwen_top_k(x[t], router, D, E, k, True)
        if mode == "underflow":
            assert np.count_nonzero(O.softmax(ora["logits"])) < k  # the corner is exercised
        assert np.array_equal(gpu["ids"][t], ora["ids"]), (list(gpu["ids"][t]), list(ora["ids"]))
        assert rel_l2(gpu["logits"][t], ora["logits"]) <= 1e-5
        # Logits of magnitude ~1e3 move the weights by the GEMV's rounding, so
        # the selection is also checked on the device's own logits, exactly.
        ids_own, w_own = O.route_top_k(gpu["logits"][t], k, True)
        assert np.array_equal(gpu["ids"][t], ids_own)
        assert max_abs(gpu["weights"][t], w_own) <= 1e-6
        if mode != "underflow":
            assert max_abs(gpu["weights"][t], ora["weights"]) <= 1e-6


def test_moe_rejects_invalid(ctx):
    g = osm_hip.geometry(2048, 512, 64, osm_hip.BF16)
    r = np.zeros(16 * 2048, np.uint16)
    with pytest.raises(osm_hip.OsmError):
        osm_hip.MoeLayer(ctx, g, 16, 17, r)  # top_k > experts
    bad = r.copy()
    bad[5] = 0x7F80  # +inf
    with pytest.raises(osm_hip.OsmError):
        osm_hip.MoeLayer(ctx, g, 16, 2, bad)
    moe = osm_hip.MoeLayer(ctx, g, 16, 2, r, max_tokens=1)
    slab = osm_hip.ExpertSlab(ctx, g, 1, 16)
    with pytest.raises(osm_hip.OsmError):
        moe.run_slab(slab, 0, np.full((1, 2048), np.nan, np.float32))
    with pytest.raises(osm_hip.OsmError):
        moe.run_slab(slab, 0, np.zeros((2, 2048), np.float32))  # more tokens than max_tokens


@pytest.mark.parametrize("chained", [False, True])
def test_decode_graph_replays_match_eager(ctx, chained):
    # A decode step over three layers captured into a HIP graph: every replay,
    # with fresh input contents and eager work and synchronisation in between,
    # must give the bits of the same step enqueued eagerly (the kernels are
    # deterministic: no atomics, fixed reduction orders).
    seed, D, I, G, E, k, L, B = 11, 256, 128, 64, 64, 4, 3, 2
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    slab = osm_hip.ExpertSlab(ctx, g, L, E)
    slab.synthesize(seed)
    layers = [osm_hip.MoeLayer(ctx, g, E, k, O.synth_router_bf16(seed, l, E, D), osm_hip.BF16,
                               O.synth_shared_gate_bf16(seed, l, D), O.synth_norm_weight(seed, l, D),
                               O.synth_expert_blob(seed, l, O.SHARED_EXPERT_ID, D, I, G), max_tokens=B)
              for l in range(L)]
    n = (1 if chained else L) * B * D
    x, y, scratch, x_ref, y_ref = (ctx.alloc(L * B * D * 4) for _ in range(5))
    graph = osm_hip.decode_graph(ctx, layers, list(range(L)), slab, x.ptr, y.ptr, scratch.ptr, B, chained)
    rng = np.random.default_rng(seed)
    for _ in range(3):
        xin = rng.normal(0, 1, n).astype(np.float32)
        x.upload(xin)
        graph.launch()
        got = y.download(np.float32, n)
        x_ref.upload(xin)
        osm_hip.decode_layers(ctx, layers, list(range(L)), slab, x_ref.ptr, y_ref.ptr, scratch.ptr, B, chained)
        ref = y_ref.download(np.float32, n)
        assert np.all(np.isfinite(ref))
        assert np.array_equal(got, ref)


def test_captured_phases_match_decode(ctx):
    # The three kernels of one decode, launched one by one inside a capture
    # and replayed, give the bits of decode_device.
    seed, D, I, G, E, k = 12, 256, 128, 64, 64, 4
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    slab = osm_hip.ExpertSlab(ctx, g, 1, E)
    slab.synthesize(seed)
    moe = osm_hip.MoeLayer(ctx, g, E, k, O.synth_router_bf16(seed, 0, E, D), osm_hip.BF16,
                           O.synth_shared_gate_bf16(seed, 0, D), None,
                           O.synth_expert_blob(seed, 0, O.SHARED_EXPERT_ID, D, I, G), max_tokens=1)
    x, y, y_ref = (ctx.alloc(D * 4) for _ in range(3))
    with ctx.capture() as cap:
        for phase in (0, 1, 2):
            moe.launch_phase(slab, 0, x.ptr, y.ptr, 1, False, phase)
    rng = np.random.default_rng(seed)
    for _ in range(2):
        x.upload(rng.normal(0, 1, D).astype(np.float32))
        cap.graph.launch()
        got = y.download(np.float32, D)
        moe.decode_device(slab, 0, x.ptr, y_ref.ptr, 1)
        assert np.array_equal(got, y_ref.download(np.float32, D))
