"""MLX affine 8-bit router and shared gate, as real checkpoints store
mlp.gate and shared_expert_gate (checkpoint_sparse_moe_test.cpp:455-460; the
reference dequantises both at load, checkpoint_sparse_moe.cpp:59-90 and
159-162, and routes on the fp32 values). Here they stay 8-bit in HBM and
the router kernel dequantises in registers with the reference's rounding
(product, then bias), so a layer built from the 8-bit modules must give the
same bits as one built from their fp32 dequantisation, on every path; and
the oracle (pinned dequant + router) sets the bars against the reference."""

import numpy as np
import pytest

import oracle as O
import osm_hip
from helpers import max_abs, rel_l2

pytestmark = pytest.mark.gpu


def quantize_q8(w, group, rng):
    """Per-group affine 8-bit: scale = (max - min) / 255, bias = min (fixture
    generation only; the values under test are the dequantised ones)."""
    rows, cols = w.shape
    g = w.reshape(rows, cols // group, group)
    lo, hi = g.min(axis=2), g.max(axis=2)
    scale = np.where(hi > lo, (hi - lo) / 255.0, 1.0).astype(np.float32)
    q = np.clip(np.rint((g - lo[..., None]) / scale[..., None]), 0, 255).astype(np.uint32).reshape(rows, cols)
    packed = (q[:, 0::4] | (q[:, 1::4] << 8) | (q[:, 2::4] << 16) | (q[:, 3::4] << 24)).astype(np.uint32)
    return packed, scale, lo.astype(np.float32)


def dequant(packed, scales, biases, group):
    rows, words = packed.shape
    return O.dequantize_affine_rows(packed, rows, words, scales, biases, bits=8, group_size=group).reshape(rows, -1)


def build(ctx, seed, D, I, G, E, k, group, max_tokens):
    rng = np.random.default_rng(seed)
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    slab = osm_hip.ExpertSlab(ctx, g, 1, E)
    slab.synthesize(seed)
    shared = O.synth_expert_blob(seed, 0, O.SHARED_EXPERT_ID, D, I, G)
    rq = quantize_q8(rng.normal(0, 0.9 / np.sqrt(D), (E, D)).astype(np.float32), group, rng)
    sq = quantize_q8(rng.normal(0, 1.0 / np.sqrt(D), (1, D)).astype(np.float32), group, rng)
    r32, s32 = dequant(*rq, group), dequant(*sq, group).reshape(-1)
    q8 = osm_hip.MoeLayer(ctx, g, E, k, rq + (group,), osm_hip.AFFINE_Q8, sq + (group,), None, shared,
                          max_tokens=max_tokens)
    f32 = osm_hip.MoeLayer(ctx, g, E, k, r32, osm_hip.F32, s32, None, shared, max_tokens=max_tokens)
    return g, slab, shared, q8, f32, r32, s32


def same(a, b):
    for key in ("ids", "weights", "logits", "shared_gate", "out"):
        assert np.array_equal(a[key], b[key]), key


@pytest.mark.parametrize("group", [64, 4])
def test_q8_router_decode_matches_fp32_and_oracle(ctx, group):
    seed, D, I, G, E, k = 61, 512, 256, 64, 128, 8
    g, slab, shared, q8, f32, r32, s32 = build(ctx, seed, D, I, G, E, k, group, 4)
    x = O.synth_tokens(seed, 0, 4, D)
    for tokens in (1, 4):  # batch 1 and the per-token kernels of a small batch
        a = q8.run_slab(slab, 0, x[:tokens])
        b = f32.run_slab(slab, 0, x[:tokens])
        same(a, b)
    blobs = [O.synth_expert_blob(seed, 0, e, D, I, G) for e in range(E)]
    for t in range(4):
        ora = O.qwen_sparse_moe(x[t], r32, blobs, shared, s32, D, I, G, O.META_BF16, k)
        assert np.array_equal(a["ids"][t], ora["ids"])
        assert max_abs(a["weights"][t], ora["weights"]) <= 1e-6
        assert rel_l2(a["out"][t], ora["out"]) <= 1e-3


def test_q8_router_grouped_and_prefill(ctx):
    # 48 fp32 tokens through the grouped experts (the per-token router kernel
    # serves a non-bf16 router) and a bf16 prefill chunk (widened for it).
    seed, D, I, G, E, k, T = 62, 512, 256, 64, 64, 6, 48
    g, slab, shared, q8, f32, r32, s32 = build(ctx, seed, D, I, G, E, k, 64, T)
    x = O.synth_tokens(seed, 100, T, D)
    for m in (q8, f32):
        m.set_path(osm_hip.PATH_GROUPED)
    same(q8.run_slab(slab, 0, x), f32.run_slab(slab, 0, x))
    u = x.view(np.uint32)
    bits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    xb, ya, yb = ctx.alloc(T * D * 2), ctx.alloc(T * D * 4), ctx.alloc(T * D * 4)
    xb.upload(bits)
    q8.prefill_device(slab, 0, xb.ptr, ya.ptr, T)
    f32.prefill_device(slab, 0, xb.ptr, yb.ptr, T)
    got, ref = ya.download(np.float32, T * D), yb.download(np.float32, T * D)
    assert np.array_equal(got, ref)
    xw = (bits.astype(np.uint32) << 16).view(np.float32).reshape(T, D)
    f32.set_path(osm_hip.PATH_PER_TOKEN)
    per = f32.run_slab(slab, 0, xw)
    assert rel_l2(got, per["out"].reshape(-1)) <= 2e-5


def test_q8_router_rejected_shapes(ctx):
    D, I, G, E, k = 256, 128, 64, 16, 4
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    shared = O.synth_expert_blob(1, 0, O.SHARED_EXPERT_ID, D, I, G)
    rng = np.random.default_rng(3)

    def q8(rows, group, bad_scale=False):
        packed = rng.integers(0, 2**32, (rows, D // 4), dtype=np.uint64).astype(np.uint32)
        scales = np.full((rows, D // group), 1e-3, np.float32)
        if bad_scale:
            scales[0, 0] = np.inf
        return packed, scales, np.zeros((rows, D // group), np.float32), group

    ok = osm_hip.MoeLayer(ctx, g, E, k, q8(E, 32), osm_hip.AFFINE_Q8, q8(1, 32), None, shared)
    del ok
    for router, sg in ((q8(E, 6), q8(1, 6)),          # not a multiple of 4
                       (q8(E, 24), q8(1, 24)),        # does not divide hidden
                       (q8(E, 32), q8(1, 64)),        # router and gate groups differ
                       (q8(E, 32, True), q8(1, 32)),  # a non-finite dequantised weight
                       (q8(E, 32), q8(1, 32, True))):
        with pytest.raises(osm_hip.OsmError):
            osm_hip.MoeLayer(ctx, g, E, k, router, osm_hip.AFFINE_Q8, sg, None, shared)
