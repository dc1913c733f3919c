"""Routing parity at volume: thousands of seeded tokens at the Qwen3-Next
shape (hidden 2048, 512 experts, top-10, bf16 router), every token's ids
against the oracle's restatement of route_qwen_top_k_cpu
(src/model/qwen_router.cpp:11-94 over src/cpu/reference_ops.cpp:85-212),
through each way the device selects:

- the per-token kernels below 12 tokens, where every gate/up workgroup
  selects its token's picks from the router's logits and bounds;
- the per-token kernels from 12 tokens, where the selection kernel selects
  once per token and gate/up reads the published slots;
- the same with the sublayer's RMSNorm, whose exact path also recomputes
  the norm's scale in the reference's order;
- the grouped prefill, whose logits and bounds come from the router GEMM.

About 4% of the per-token selections (14% behind the router GEMM) are not
proven by the bounds and take the exact path, so each case takes it dozens
of times; the routing counters must show that it did. The weights must
agree with the oracle's within what the logits' rounding explains: a weight
is exp(l_i - m) / sum over the picks of exp(l_j - m), so a logit error d
moves it by at most 2 w d.
"""

import numpy as np
import pytest

import oracle as O
import osm_hip
from test_gpu_moe import QwenLayer

pytestmark = pytest.mark.gpu


def _check_tokens(L, x_route, routing, first):
    router = O.bf16_bits_to_f32(L.router_bits)
    for t in range(x_route.shape[0]):
        ora = O.route_qwen_top_k(x_route[t], router, L.D, L.E, L.k, True)
        ids = ora["ids"]
        assert np.array_equal(routing["ids"][t], ids), first + t
        d = float(np.max(np.abs(routing["logits"][t][ids].astype(np.float64) - ora["logits"][ids])))
        dw = float(np.max(np.abs(routing["weights"][t].astype(np.float64) - ora["weights"])))
        assert dw <= 1e-6 + 2.0 * float(np.max(ora["weights"])) * d, (first + t, dw, d)


@pytest.mark.parametrize("per_call,calls,sublayer", [(8, 384, False), (32, 96, False), (8, 192, True), (32, 48, True)],
                         ids=["gate_up_selects", "selection_kernel", "gate_up_selects_rmsnorm",
                              "selection_kernel_rmsnorm"])
def test_per_token_routing_sweep(ctx, per_call, calls, sublayer):
    seed = 611 + per_call + (7 if sublayer else 0)
    L = QwenLayer(ctx, seed, max_tokens=per_call, norm=sublayer)
    L.moe.set_path(osm_hip.PATH_PER_TOKEN)
    xb, yb = ctx.alloc(per_call * L.D * 4), ctx.alloc(per_call * L.D * 4)
    L.moe.routing_stats(reset=True)
    for c in range(calls):
        x = O.synth_tokens(seed, 10000 + c * per_call, per_call, L.D)
        xb.upload(x)
        L.moe.decode_device(L.slab, 0, xb.ptr, yb.ptr, per_call, sublayer=sublayer)
        routing = L.moe.routing(per_call)
        x_route = O.rms_norm(x, per_call, L.D, L.norm_w, 1e-6) if sublayer else x
        _check_tokens(L, x_route.reshape(per_call, L.D), routing, c * per_call)
    st = L.moe.routing_stats()
    print(f"per-token sweep, {per_call} tokens per call, sublayer={sublayer}: {st}")
    assert st["selections"] == per_call * calls, st
    assert st["exact"] >= 20, st  # the exact path ran, and agreed every time


def test_prefill_routing_sweep(ctx):
    T, chunks, seed = 512, 4, 633
    L = QwenLayer(ctx, seed, max_tokens=T)
    xb, yb = ctx.alloc(T * L.D * 2), ctx.alloc(T * L.D * 4)
    L.moe.routing_stats(reset=True)
    for c in range(chunks):
        xf = O.synth_tokens(seed, 20000 + c * T, T, L.D)
        u = xf.view(np.uint32)
        bits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        xb.upload(bits)
        L.moe.prefill_device(L.slab, 0, xb.ptr, yb.ptr, T)
        routing = L.moe.routing(T)
        xw = (bits.astype(np.uint32) << 16).view(np.float32)
        _check_tokens(L, xw, routing, c * T)
    st = L.moe.routing_stats()
    print(f"prefill sweep, {chunks} chunks of {T} tokens: {st}")
    assert st["selections"] == T * chunks and st["exact"] >= 50, st
