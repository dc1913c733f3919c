"""The decode entry point that allocates nothing, through the C ABI.

osm_moe_layer_decode_device_static runs the per-token kernels with their
routing workspace in the library's fixed per-device array. Its output must be
the bits of osm_moe_layer_decode_device (same kernels, workspace in the
layer) on the same inputs: two calls in a row, the second with fewer tokens
(so the array holds the first call's routing when the second starts), in the
MoE and the sublayer form, at the Qwen3-Next shape. The selection runs in its
own launch from 12 tokens on and inside gate/up below, so the two calls take
both routes through the kernels."""

import numpy as np
import pytest

import oracle as O
import osm_hip

pytestmark = pytest.mark.gpu

SEED, D, I, G, E, K = 91, 2048, 512, 64, 512, 10


@pytest.fixture(scope="module")
def model(ctx):
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    slab = osm_hip.ExpertSlab(ctx, g, 1, E)
    slab.synthesize(SEED)
    moe = osm_hip.MoeLayer(ctx, g, E, K, O.synth_router_bf16(SEED, 0, E, D), osm_hip.BF16,
                           O.synth_shared_gate_bf16(SEED, 0, D), O.synth_norm_weight(SEED, 0, D),
                           O.synth_expert_blob(SEED, 0, O.SHARED_EXPERT_ID, D, I, G), max_tokens=32)
    moe.set_path(osm_hip.PATH_PER_TOKEN)
    return slab, moe


@pytest.mark.parametrize("sublayer", [False, True])
def test_static_decode_matches_decode_device(ctx, model, sublayer):
    slab, moe = model
    assert moe.static_tokens_capacity == 119  # 4 MiB over this shape's per-token workspace
    x, y_ref, y = (ctx.alloc(32 * D * 4) for _ in range(3))
    for n, first in ((20, 0), (3, 100)):
        print(f"[no-alloc] sublayer={sublayer} tokens={n}", flush=True)
        x.upload(O.synth_tokens(SEED, first, n, D).reshape(-1))
        moe.decode_device(slab, 0, x.ptr, y_ref.ptr, n, sublayer=sublayer)
        moe.decode_device_static(slab, 0, x.ptr, y.ptr, n, sublayer=sublayer)
        ref = y_ref.download(np.float32, n * D)
        got = y.download(np.float32, n * D)
        assert np.all(np.isfinite(ref))
        assert np.array_equal(got, ref), (sublayer, n)
    # The static call's routing is not kept, so the query refuses it until
    # the layer's next other call.
    with pytest.raises(osm_hip.OsmError) as e:
        moe.routing(3)
    assert e.value.status == osm_hip.OSM_E_INVALID and "without allocation" in e.value.diagnostic
    moe.decode_device(slab, 0, x.ptr, y_ref.ptr, 3, sublayer=sublayer)
    assert moe.routing(3)["ids"].shape == (3, K)


def test_static_decode_rejects_beyond_capacity(ctx, model):
    slab, moe = model
    x, y = ctx.alloc(4 * D * 4), ctx.alloc(4 * D * 4)
    with pytest.raises(osm_hip.OsmError) as e:
        moe.decode_device_static(slab, 0, x.ptr, y.ptr, moe.static_tokens_capacity + 1)
    assert "static_tokens_capacity" in e.value.diagnostic
    with pytest.raises(osm_hip.OsmError):
        moe.decode_device_static(slab, 0, x.ptr, y.ptr, 0)
