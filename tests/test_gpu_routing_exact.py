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


def test_logits_one_or_two_ulps_apart(ctx):
    # Logits 2.5e-7..4.5e-7 apart (one or two ulps of a logit near 2): the
    # exact path ranks them by the reference's exps, with the host libm's
    # bits, and any adjacent pair close enough for the probabilities to tie
    # goes to the recompute over every expert. Ids are the oracle's.
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
    assert st["exact"] == 1, st


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


# ---------------------------------------------------------------------------
# Probabilities that tie although the logits differ.
#
# The reference's probabilities are p = fl(e / S), e = std::exp(fl(L - m))
# (the host libm's expf) and S the fp32 sum of every e in id order, ranked
# with the lower id first among equal p (reference_ops.cpp:135-196). Two
# different logits can give one p in three ways, and the router below
# builds each with the lower logit on the lower id, where the reference puts
# the LOWER logit first:
#   (a) fl(L - m) differs but the two exps round to one float;
#   (b) fl(L - m) itself rounds two logits to one key;
#   (c) the exps are one ulp apart but e_a / S and e_b / S round to one float
#       (inside the picks, and for the k-th pick against the (k+1)-th, where
#       the tie decides which of the two is picked);
# plus (d) exps one ulp apart whose quotients do not tie (the higher logit
# first, as usual). Logits are set exactly: the input is 1, 2^-8, 2^-16 in
# its first three columns and 0 elsewhere, and each router row holds bf16
# w0, w1, w2 with w0 + w1 2^-8 + w2 2^-16 the target, every partial sum
# exact in fp32.

def _libm_expf():
    import ctypes
    import ctypes.util
    f = ctypes.CDLL(ctypes.util.find_library("m")).expf
    f.restype = ctypes.c_float
    f.argtypes = [ctypes.c_float]
    return lambda v: np.float32(f(float(v)))


def _bf16_rne(v):
    b = int(np.array([v], np.float32).view(np.uint32)[0])
    return (b + 0x7FFF + ((b >> 16) & 1)) >> 16


def _bf16_val(bits):
    return float(np.array([bits << 16], np.uint32).view(np.float32)[0])


def _exact_logit_row(target):
    """bf16 (w0, w1, w2) with fl(fl(w0 + w1 2^-8) + w2 2^-16) == target."""
    t = float(np.float32(target))
    w0 = _bf16_rne(t)
    r1 = t - _bf16_val(w0)
    w1 = _bf16_rne(r1 * 256.0)
    r2 = r1 - _bf16_val(w1) / 256.0
    w2 = _bf16_rne(r2 * 65536.0)
    got = np.float32(np.float32(_bf16_val(w0)) + np.float32(_bf16_val(w1) / 256.0))
    got = np.float32(got + np.float32(_bf16_val(w2) / 65536.0))
    assert got == np.float32(t), (target, got)
    return w0, w1, w2


def _softmax_sum(logits, expf):
    m = np.float32(np.max(logits))
    s = np.float32(0.0)
    for v in logits:
        s = np.float32(s + expf(np.float32(v - m)))
    return s


def tie_router(rng):
    """(router bits [E, D], f32 router, x, pairs): pairs maps each case to its
    (lower id, higher id) with the lower logit on the lower id."""
    expf = _libm_expf()
    ulp24 = 2.0 ** -24
    logits = np.float32(-1.0) - np.float32(2.0) * rng.random(E).astype(np.float32)  # [-3, -1)
    ids = rng.permutation(E)
    top, rest = ids[:16], ids[16:]
    lid = lambda a, b: (int(min(a, b)), int(max(a, b)))
    m_id = int(top[0])
    logits[m_id] = 1.0
    pairs = {}
    # (a) distinct keys, equal exps, near 0.70 (keys 2^-24 apart, exps 0.74 ulp apart).
    base = 0.70
    for j in range(4096):
        lb = np.float32(base + j * ulp24)
        la = np.float32(lb + ulp24)
        xa, xb = np.float32(la - 1.0), np.float32(lb - 1.0)
        if xa != xb and expf(xa) == expf(xb):
            break
    else:
        raise AssertionError("no exp tie found")
    lo, hi = lid(top[1], top[2])
    logits[lo], logits[hi] = lb, la
    pairs["exp_tie"] = (lo, hi)
    # (b) one key from two logits near 0.45 (logits 2^-25 apart, keys 2^-24 apart).
    for j in range(4096):
        lb = np.float32(0.45 + j * 2.0 ** -25)
        la = np.float32(lb + 2.0 ** -25)
        if la != lb and np.float32(la - 1.0) == np.float32(lb - 1.0):
            break
    else:
        raise AssertionError("no key tie found")
    lo, hi = lid(top[3], top[4])
    logits[lo], logits[hi] = lb, la
    pairs["key_tie"] = (lo, hi)

    # (c), (d): exps one ulp apart, with S over the final logits.
    def one_ulp_pairs(start):
        j = 0
        while True:
            lb = np.float32(start + j * 2.0 ** -24)
            la = np.float32(lb + 2.0 ** -24)
            eb, ea = expf(np.float32(lb - 1.0)), expf(np.float32(la - 1.0))
            if ea == np.nextafter(eb, np.float32(1.0)):
                yield lb, la, eb, ea
            j += 1

    slots = {"quot_nontie": (top[5], top[6], 0.235), "quot_tie": (top[7], top[8], 0.21),
             "boundary_tie": (top[9], top[10], 0.15)}
    for name, (a, b, _) in slots.items():
        pairs[name] = lid(a, b)
    gens = {name: one_ulp_pairs(start) for name, (_, _, start) in slots.items()}
    cur = {name: next(g) for name, g in gens.items()}
    for _ in range(400):
        for name, (lb, la, _, _) in cur.items():
            lo, hi = pairs[name]
            logits[lo], logits[hi] = lb, la
        s = _softmax_sum(logits, expf)
        want = {"quot_nontie": False, "quot_tie": True, "boundary_tie": True}
        ok = True
        for name, (lb, la, eb, ea) in cur.items():
            if (np.float32(ea / s) == np.float32(eb / s)) != want[name]:
                cur[name] = next(gens[name])
                ok = False
        if ok:
            break
    else:
        raise AssertionError("no quotient ties found")
    x = np.zeros(D, np.float32)
    x[0], x[1], x[2] = 1.0, 2.0 ** -8, 2.0 ** -16
    bits = bf16_bits(rng.normal(0, 0.02, (E, D)).astype(np.float32))
    for e in range(E):
        bits[e, 0], bits[e, 1], bits[e, 2] = _exact_logit_row(logits[e])
    return bits, bf16_to_f32(bits), x, pairs, logits


def test_probability_ties_decided_as_the_reference_does(ctx):
    # Every kind of tie above, with the lower logit on the lower id, through
    # every path: one token (selection inside gate/up), 16 tokens (the select
    # kernel), grouped at 16 (per-token router) and 24 (router GEMM). Ids are
    # the oracle's bit for bit; the three one-ulp pairs (higher id first by
    # exp) send every selection to the recompute over every expert.
    rng = np.random.default_rng(11)
    bits, router_f, x, pairs, logits = tie_router(rng)
    ora = O.route_qwen_top_k(x, router_f, D, E, K, True)
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    blob = random_blob(rng, D, I, G, O.META_BF16)[0]
    slab = osm_hip.ExpertSlab(ctx, g, 1, E)
    for e in range(E):
        slab.upload(0, e, blob)
    moe = osm_hip.MoeLayer(ctx, g, E, K, bits, osm_hip.BF16, max_tokens=24)
    for path, T in [(osm_hip.PATH_PER_TOKEN, 1), (osm_hip.PATH_PER_TOKEN, 16), (osm_hip.PATH_GROUPED, 16),
                    (osm_hip.PATH_GROUPED, 24)]:
        moe.routing_stats(reset=True)
        moe.set_path(path)
        gpu = moe.run_slab(slab, 0, np.tile(x, (T, 1)))
        for t in range(T):
            assert np.array_equal(gpu["ids"][t], ora["ids"]), (path, T, t, list(gpu["ids"][t]), list(ora["ids"]))
            assert_weights(gpu["weights"][t], gpu["logits"][t], gpu["ids"][t], ora["weights"], ora["logits"])
        st = moe.routing_stats()
        assert st["selections"] == T and st["exact"] == T and st["exact_all"] == T, (path, T, st)
        assert st["near_ties"] == 3 * T, (path, T, st)


def test_device_exp_keys_equal_host_libm(ctx):
    # The selection's exp (osm_libm_expf as compiled for gfx950) over every
    # float <= 0, against std::exp(float) of this host: checksums of 2^16
    # results at a time (sum of bits * (2 i + 1): any single wrong result
    # changes its block's sum).
    first, count, block = 0x80000000, 0x7F800001, 1 << 16
    dev = osm_hip.libm_expf_checksums(ctx, first, count, block)
    host = O.libm_expf_checksums(first, count, block)
    bad = np.nonzero(dev != host)[0]
    assert bad.size == 0, [hex(first + int(b) * block) for b in bad[:8]]
