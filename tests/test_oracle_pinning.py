"""Pins the CPU oracle (oracle/osm_oracle.cpp) before it is trusted as the
checker: the reference's known-answer tests, closed forms and brute force,
and -- where the reference checkout was available at build time -- the
reference's own CPU functions compiled into oracle/_ref (bit-exact)."""

import math

import numpy as np
import pytest

import oracle as O
from helpers import bf16_bits, bf16_to_f32, pack_q4

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference checkout)")


# ---- reference_ops.cpp: dequantize_affine_rows ----------------------------------------
def test_q4_affine_kat():
    # tests/cpu_reference_test.cpp:48-71: nibbles 0..7, scale 2, bias -1 -> 2i-1.
    word = sum(i << (4 * i) for i in range(8))
    out = O.dequantize_affine_rows([word], 1, 1, [2.0], [-1.0], bits=4, group_size=8)
    assert np.array_equal(out, np.array([2 * i - 1 for i in range(8)], np.float32))


def test_q8_affine_kat():
    # tests/cpu_reference_test.cpp:73-93.
    word = 2 | (4 << 8) | (6 << 16) | (8 << 24)
    out = O.dequantize_affine_rows([word], 1, 1, [0.5], [1.0], bits=8, group_size=4)
    assert np.array_equal(out, np.array([2.0, 3.0, 4.0, 5.0], np.float32))


def test_dequant_exhaustive_nibbles_closed_form():
    # Every nibble value in every lane: value = fl(fl(s*q) + b), column = 8*word + lane.
    rng = np.random.default_rng(1)
    q = np.zeros((16, 8 * 16), np.uint32)
    for v in range(16):
        for lane in range(8):
            q[v, lane * 16 + v] = v  # distinct lanes/words per value
    q = (q + rng.integers(0, 16, q.shape, dtype=np.uint32) * (q == 0)) & 0xF
    packed = pack_q4(q)
    s = rng.normal(0, 0.05, (16, 2)).astype(np.float32)
    b = rng.normal(0, 0.3, (16, 2)).astype(np.float32)
    out = O.dequantize_affine_rows(packed, 16, 16, s, b, 4, 64).reshape(16, 128)
    expect = (np.repeat(s, 64, 1) * q.astype(np.float32)).astype(np.float32) + np.repeat(b, 64, 1)
    assert np.array_equal(out, expect.astype(np.float32))


@pytest.mark.parametrize("bits,group", [(3, 8), (4, 0), (4, 3)])
def test_dequant_rejects_invalid(bits, group):
    # cpu_reference_test.cpp:149-166 (3-bit) and the group checks of reference_ops.cpp:18-42.
    with pytest.raises(O.OracleError) as e:
        O.dequantize_affine_rows([0], 1, 1, [1.0], [0.0], bits=bits, group_size=group)
    assert e.value.code == 1


@needs_ref
def test_dequant_matches_reference_build():
    rng = np.random.default_rng(2)
    packed = rng.integers(0, 2**32, (33, 64), dtype=np.uint64).astype(np.uint32)
    s = rng.normal(0, 0.02, (33, 8)).astype(np.float32)
    b = rng.normal(0, 0.2, (33, 8)).astype(np.float32)
    a = O.dequantize_affine_rows(packed, 33, 64, s, b, 4, 64)
    r = O.dequantize_affine_rows(packed, 33, 64, s, b, 4, 64, impl="ref")
    assert np.array_equal(a, r)


# ---- matvec ---------------------------------------------------------------------------------
def test_matvec_kat():
    # cpu_reference_test.cpp:95-104.
    y = O.matvec_row_major([1, 2, -1, 3], 2, 2, [4, 5])
    assert np.array_equal(y, np.array([14.0, 11.0], np.float32))


def test_matvec_sequential_order_and_fp64():
    rng = np.random.default_rng(3)
    w = rng.normal(0, 1, (5, 300)).astype(np.float32)
    x = rng.normal(0, 1, 300).astype(np.float32)
    y = O.matvec_row_major(w, 5, 300, x)
    # Bit-exact against a left-to-right fp32 loop (numpy scalars, no fusion).
    for r in range(5):
        acc = np.float32(0)
        for c in range(300):
            acc = np.float32(acc + np.float32(w[r, c] * x[c]))
        assert y[r] == acc
    # And close to the exact sum.
    exact = w.astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(y - exact)) < 1e-4


@needs_ref
def test_matvec_matches_reference_build():
    rng = np.random.default_rng(4)
    w = rng.normal(0, 1, (64, 2048)).astype(np.float32)
    x = rng.normal(0, 1, 2048).astype(np.float32)
    assert np.array_equal(O.matvec_row_major(w, 64, 2048, x), O.matvec_row_major(w, 64, 2048, x, impl="ref"))


# ---- RMSNorm --------------------------------------------------------------------------------
def test_rmsnorm_kat():
    # cpu_reference_test.cpp:106-112.
    out = O.rms_norm([3.0, 4.0], 1, 2, [2.0, 0.5], 0.0)
    base = math.sqrt((9 + 16) / 2)
    assert abs(out[0] - 3 / base * 2) < 1e-6 and abs(out[1] - 4 / base * 0.5) < 1e-6


@needs_ref
def test_rmsnorm_matches_reference_build():
    rng = np.random.default_rng(5)
    v = rng.normal(0, 1, 3 * 2048).astype(np.float32)
    w = (1 + rng.normal(0, 0.02, 2048)).astype(np.float32)
    assert np.array_equal(O.rms_norm(v, 3, 2048, w, 1e-6), O.rms_norm(v, 3, 2048, w, 1e-6, impl="ref"))


# ---- softmax / top-k ---------------------------------------------------------------------------
def _brute_top_k(logits, k):
    p = np.asarray(O.softmax(logits), np.float32)
    order = sorted(range(len(p)), key=lambda i: (-float(p[i]), i))[:k]
    return np.array(order, np.uint32), p[order]


def test_top_k_kat():
    # cpu_reference_test.cpp:115-136.
    ids, pr = O.route_top_k([0, 1, 2, 3], 2, False)
    assert list(ids) == [3, 2]
    probs = O.softmax([0, 1, 2, 3])
    assert abs(pr[0] - probs[3]) < 1e-6 and abs(pr[1] - probs[2]) < 1e-6
    ids, pr = O.route_top_k([0, 1, 2, 3], 2, True)
    assert list(ids) == [3, 2] and abs(pr.sum() - 1) < 1e-6


@pytest.mark.parametrize("seed", range(6))
def test_top_k_brute_force_with_ties(seed):
    rng = np.random.default_rng(100 + seed)
    # Few distinct values -> many exact ties: lower id must win (reference_ops.cpp:170-196).
    logits = rng.integers(0, 5, 64).astype(np.float32) * np.float32(0.25)
    for k in (1, 3, 10, 64):
        ids, pr = O.route_top_k(logits, k, False)
        bids, bpr = _brute_top_k(logits, k)
        assert np.array_equal(ids, bids) and np.array_equal(pr, bpr)


@needs_ref
@pytest.mark.parametrize("seed", range(4))
def test_top_k_matches_reference_build(seed):
    rng = np.random.default_rng(200 + seed)
    logits = rng.normal(0, 1, 512).astype(np.float32)
    logits[::7] = logits[3]  # ties
    for norm in (False, True):
        a = O.route_top_k(logits, 10, norm)
        r = O.route_top_k(logits, 10, norm, impl="ref")
        assert np.array_equal(a[0], r[0]) and np.array_equal(a[1], r[1])


# ---- router (qwen_router.cpp) ---------------------------------------------------------------------
def test_router_kats():
    # tests/qwen_router_test.cpp:51-179.
    r = O.route_qwen_top_k([1.0], [1, 2, 3, 4], 1, 4, 2, True)
    e = [math.exp(v) for v in (1, 2, 3, 4)]
    tot = sum(e)
    assert list(r["ids"]) == [3, 2]
    assert abs(r["mass"] - (e[3] + e[2]) / tot) < 1e-6
    assert abs(r["weights"][0] - e[3] / (e[3] + e[2])) < 1e-6
    assert abs(r["weights"][1] - e[2] / (e[3] + e[2])) < 1e-6
    raw = O.route_qwen_top_k([1.0], [1, 2, 3, 4], 1, 4, 2, False)
    assert list(raw["ids"]) == [3, 2]
    assert abs(raw["weights"][0] - e[3] / tot) < 1e-6 and abs(raw["weights"][1] - e[2] / tot) < 1e-6
    assert raw["mass"] < 1.0
    tie = O.route_qwen_top_k([1.0], [5, 5, 1, 0], 1, 4, 1, True)
    assert list(tie["ids"]) == [0] and abs(tie["weights"][0] - 1) < 1e-6
    ramp = O.route_qwen_top_k([1.0], np.arange(512, dtype=np.float32) * np.float32(0.01), 1, 512, 10, True)
    assert list(ramp["ids"]) == [511 - i for i in range(10)]
    assert abs(ramp["weights"].sum() - 1) < 1e-5
    with pytest.raises(O.OracleError):
        O.route_qwen_top_k([1.0], [1.0, 2.0], 1, 4, 2, True)


def test_router_rejects_non_finite():
    with pytest.raises(O.OracleError):
        O.route_qwen_top_k([float("nan")], [1, 2, 3, 4], 1, 4, 2, True)
    with pytest.raises(O.OracleError):
        O.route_qwen_top_k([1.0], [1, float("inf"), 3, 4], 1, 4, 2, True)


@needs_ref
@pytest.mark.parametrize("seed", range(3))
def test_router_matches_reference_build(seed):
    hidden = O.synth_tokens(seed, 0, 1, 2048)[0]
    router = O.bf16_bits_to_f32(O.synth_router_bf16(seed, 0, 512, 2048))
    a = O.route_qwen_top_k(hidden, router, 2048, 512, 10, True)
    r = O.route_qwen_top_k(hidden, router, 2048, 512, 10, True, impl="ref")
    for key in ("logits", "ids", "weights"):
        assert np.array_equal(a[key], r[key])
    assert a["mass"] == r["mass"]


# ---- shared expert ---------------------------------------------------------------------------------
def _shared_fixture():
    # tests/shared_expert_test.cpp:33-55.
    hidden, inter = 8, 4
    x = np.array([(i - 3) * 0.25 for i in range(hidden)], np.float32)
    gate = np.array([((i % 9) - 4) * 0.0625 for i in range(inter * hidden)], np.float32)
    up = np.array([(((i * 3) % 11) - 5) * 0.05 for i in range(inter * hidden)], np.float32)
    down = np.array([(((i * 5) % 13) - 6) * 0.04 for i in range(hidden * inter)], np.float32)
    scalar = np.array([((i % 5) - 2) * 0.125 for i in range(hidden)], np.float32)
    return hidden, inter, x, gate, up, down, scalar


# ---- reference_ops.cpp: sigmoid / silu / swiglu -------------------------------------------
def test_swiglu_kat_and_closed_form():
    # tests/cpu_reference_test.cpp:138-147, and the closed forms in fp64:
    # sigmoid(v) = 1 / (1 + e^-v), silu(v) = v * sigmoid(v).
    out = O.swiglu([-1.0, 0.0, 1.0], [2.0, 3.0, 4.0])
    assert abs(out[0] - O.silu(-1.0) * 2.0) <= 1e-6 and out[1] == 0.0 and abs(out[2] - O.silu(1.0) * 4.0) <= 1e-6
    assert O.sigmoid(0.0) == 0.5
    for v in np.linspace(-30, 30, 241):
        v = float(np.float32(v))
        sig = 1.0 / (1.0 + math.exp(-v))
        assert abs(O.sigmoid(v) - sig) <= 2 * np.spacing(np.float32(sig))
        assert abs(O.silu(v) - v * sig) <= 4 * np.spacing(np.float32(abs(v * sig))) + 1e-45
    rng = np.random.default_rng(7)
    g, u = rng.normal(0, 3, 257).astype(np.float32), rng.normal(0, 1, 257).astype(np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.max(np.abs(O.swiglu(g, u) - ref)) <= 1e-6


@needs_ref
def test_swiglu_matches_reference_build():
    rng = np.random.default_rng(8)
    g, u = rng.normal(0, 3, 1000).astype(np.float32), rng.normal(0, 1, 1000).astype(np.float32)
    assert np.array_equal(O.swiglu(g, u), O.swiglu(g, u, impl="ref"))


def test_shared_expert_closed_form():
    hidden, inter, x, gate, up, down, scalar = _shared_fixture()
    out, sg = O.run_shared_expert(x, gate, up, down, scalar, hidden, inter)
    g = gate.reshape(inter, hidden).astype(np.float64) @ x
    u = up.reshape(inter, hidden).astype(np.float64) @ x
    h = g / (1 + np.exp(-g)) * u
    y = down.reshape(hidden, inter).astype(np.float64) @ h
    s = 1 / (1 + math.exp(-float(scalar.astype(np.float64) @ x)))
    assert abs(sg - s) < 1e-7
    assert np.max(np.abs(out - y * s)) < 1e-6


@needs_ref
def test_shared_expert_matches_reference_build():
    hidden, inter, x, gate, up, down, scalar = _shared_fixture()
    a = O.run_shared_expert(x, gate, up, down, scalar, hidden, inter)
    r = O.run_shared_expert(x, gate, up, down, scalar, hidden, inter, impl="ref")
    assert np.array_equal(a[0], r[0]) and a[1] == r[1]


# ---- metadata widening (vulkan_qpack_expert.cpp:54-87) -----------------------------------------------
def test_bf16_f16_widening_exhaustive():
    bits = np.arange(65536, dtype=np.uint32)
    # Floats come back through ctypes as Python doubles, which quiets NaN
    # payloads, so NaN patterns are compared by class only.
    bf = np.array([O.bf16_to_float(int(b)) for b in bits], np.float32)
    expect_bf = (bits << 16).astype(np.uint32).view(np.float32)
    fin = ~np.isnan(expect_bf)
    assert np.array_equal(bf[fin].view(np.uint32), expect_bf[fin].view(np.uint32))
    assert np.array_equal(np.isnan(bf), np.isnan(expect_bf))
    f16 = np.array([O.f16_to_float(int(b)) for b in bits], np.float32)
    ref16 = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    finite = np.isfinite(ref16)
    assert np.array_equal(f16[finite].view(np.uint32), ref16[finite].view(np.uint32))
    assert np.array_equal(np.isnan(f16), np.isnan(ref16)) and np.array_equal(np.isinf(f16), np.isinf(ref16))


# ---- composition -------------------------------------------------------------------------------------
def _ref_projection_ptrs(blob, hidden, inter, group, meta):
    """The nine section arrays (metadata widened to fp32) the reference shim takes."""
    secs = O.blob_sections(blob, hidden, inter, group, meta)
    arrays = []
    for q, s, b in secs:
        arrays += [np.ascontiguousarray(q, np.uint32), np.ascontiguousarray(s, np.float32), np.ascontiguousarray(b, np.float32)]
    return arrays


def _ref_sparse_moe(hidden, router, blobs, shared_blob, shared_sg, h, inter, group, meta, k):
    import ctypes
    arrays = []
    table = []
    for bl in blobs:
        arr = _ref_projection_ptrs(bl, h, inter, group, meta)
        arrays.append(arr)
        table += [a.ctypes.data for a in arr]
    sh = _ref_projection_ptrs(shared_blob, h, inter, group, meta)
    tab = (ctypes.c_void_p * len(table))(*table)
    shp = (ctypes.c_void_p * 9)(*[a.ctypes.data for a in sh])
    out = np.zeros(h, np.float32)
    ids = np.zeros(k, np.uint32)
    w = np.zeros(k, np.float32)
    x, r, s = O.f32(hidden), O.f32(router), O.f32(shared_sg)
    rc = O.ref().ref_sparse_moe(O.p(x), O.p(r), len(blobs), k, ctypes.cast(tab, ctypes.c_void_p),
                                ctypes.cast(shp, ctypes.c_void_p), O.p(s), h, inter, group, O.p(out), O.p(ids), O.p(w))
    assert rc == 0, O.ref().ref_last_error()
    return out, ids, w


@needs_ref
@pytest.mark.parametrize("meta", [O.META_BF16, O.META_F32])
def test_sparse_moe_matches_reference_build(meta):
    seed, h, inter, E, k = 7, 256, 64, 12, 3
    blobs = [O.synth_expert_blob(seed, 0, e, h, inter, 64, meta) for e in range(E)]
    shared = O.synth_expert_blob(seed, 0, O.SHARED_EXPERT_ID, h, inter, 64, meta)
    router = O.bf16_bits_to_f32(O.synth_router_bf16(seed, 0, E, h))
    sg = O.bf16_bits_to_f32(O.synth_shared_gate_bf16(seed, 0, h))
    x = O.synth_tokens(seed, 0, 1, h)[0]
    a = O.qwen_sparse_moe(x, router, blobs, shared, sg, h, inter, 64, meta, k)
    r_out, r_ids, r_w = _ref_sparse_moe(x, router, blobs, shared, sg, h, inter, 64, meta, k)
    assert np.array_equal(a["ids"], r_ids)
    assert np.array_equal(a["weights"], r_w)
    assert np.array_equal(a["out"], r_out)


def test_expert_forward_fp64():
    # The composed expert MLP against an fp64 evaluation of the same math.
    seed, h, inter = 11, 256, 64
    blob = O.synth_expert_blob(seed, 0, 3, h, inter, 64, O.META_BF16)
    x = O.synth_tokens(seed, 0, 1, h)[0].astype(np.float64)
    secs = O.blob_sections(blob, h, inter, 64, O.META_BF16)

    def dense(q, s, b):
        from helpers import unpack_q4
        qq = unpack_q4(q).astype(np.float64)
        return np.repeat(s.astype(np.float64), 64, 1) * qq + np.repeat(b.astype(np.float64), 64, 1)

    g = dense(*secs[0]) @ x
    u = dense(*secs[1]) @ x
    y = dense(*secs[2]) @ (g / (1 + np.exp(-g)) * u)
    out = O.expert_forward(blob, h, inter, 64, O.META_BF16, x.astype(np.float32))
    assert np.linalg.norm(out - y) / np.linalg.norm(y) < 1e-5


def test_sublayer_is_norm_moe_residual():
    # checkpoint_moe_sublayer.cpp:138-199: out = residual + MoE(RMSNorm(residual)).
    seed, h, inter, E, k = 9, 256, 64, 8, 2
    blobs = [O.synth_expert_blob(seed, 0, e, h, inter) for e in range(E)]
    shared = O.synth_expert_blob(seed, 0, O.SHARED_EXPERT_ID, h, inter)
    router = O.bf16_bits_to_f32(O.synth_router_bf16(seed, 0, E, h))
    sg = O.bf16_bits_to_f32(O.synth_shared_gate_bf16(seed, 0, h))
    nw = O.synth_norm_weight(seed, 0, h)
    x = O.synth_tokens(seed, 0, 1, h)[0] * np.float32(3.0)
    sub = O.moe_sublayer(x, nw, 1e-6, router, blobs, shared, sg, h, inter, 64, O.META_BF16, k)
    norm = O.rms_norm(x, 1, h, nw, 1e-6)
    assert np.array_equal(sub["normalized"], norm)
    moe = O.qwen_sparse_moe(norm, router, blobs, shared, sg, h, inter, 64, O.META_BF16, k)
    assert np.array_equal(sub["out"], (x + moe["out"]).astype(np.float32))
    assert np.array_equal(sub["ids"], moe["ids"])


def test_sublayer_with_given_picks_is_the_routed_sublayer():
    # The given-picks sublayer fed the router's own picks is the routed
    # sublayer bit for bit (routed_moe.cpp:31-62 accumulates the picks in
    # order, as the routed path does), for several tokens; with the picks
    # reversed it still matches to rounding (a reordered sum), so the weights
    # and blobs are paired by pick, not by position in the expert table.
    seed, h, inter, E, k = 19, 256, 64, 16, 4
    blobs = [O.synth_expert_blob(seed, 0, e, h, inter) for e in range(E)]
    shared = O.synth_expert_blob(seed, 0, O.SHARED_EXPERT_ID, h, inter)
    router = O.bf16_bits_to_f32(O.synth_router_bf16(seed, 0, E, h))
    sg = O.bf16_bits_to_f32(O.synth_shared_gate_bf16(seed, 0, h))
    nw = O.synth_norm_weight(seed, 0, h)
    for t, x in enumerate(O.synth_tokens(seed, 0, 4, h)):
        sub = O.moe_sublayer(x, nw, 1e-6, router, blobs, shared, sg, h, inter, 64, O.META_BF16, k)
        picked = [blobs[int(e)] for e in sub["ids"]]
        got = O.moe_sublayer_picks(x, nw, 1e-6, sub["weights"], picked, shared, sg, h, inter, 64, O.META_BF16)
        assert np.array_equal(got, sub["out"]), t
        rev = O.moe_sublayer_picks(x, nw, 1e-6, sub["weights"][::-1].copy(), picked[::-1], shared, sg, h, inter, 64,
                                   O.META_BF16)
        assert np.max(np.abs(rev - sub["out"])) <= 1e-5 * np.max(np.abs(sub["out"])), t


# ---- single_expert_pilot.cpp: quantize_affine_q4_rows (a16) ------------------------------
# The reference's source needs nlohmann/json, so it is not in oracle/_ref; the
# restatement is pinned by the reference's own test and by properties that fix
# every output: the argmin of the reconstruction, exact grids, flat groups,
# halves away from zero, and the error statistics.
def test_quantizer_reference_test():
    # tests/affine_q4_quantizer_test.cpp:21-52.
    v = np.array([-1.0, -0.5, 0.0, 0.5, 1.0, 1.5, 2.0, 2.5, 3.0, 3.0, 3.0, 3.0, -2.0, -1.0, 0.0, 1.0], np.float32)
    packed, s, b, mx, mean = O.quantize_affine_q4_rows(v, 2, 8, 4)
    assert packed.size == 2 and s.size == 4 and b.size == 4 and math.isfinite(mx) and math.isfinite(mean)
    d = O.dequantize_affine_rows(packed, 2, 1, s, b, bits=4, group_size=4)
    assert abs(float(np.max(np.abs(d - v))) - mx) <= 1e-6
    with pytest.raises(O.OracleError) as e:
        O.quantize_affine_q4_rows(v, 2, 8, 3)
    assert e.value.code == 1


@pytest.mark.parametrize("group", [4, 8, 32, 64, 128])
def test_quantizer_argmin_and_statistics(group):
    rng = np.random.default_rng(group)
    rows, cols = 6, 256
    v = rng.normal(0, 0.05, (rows, cols)).astype(np.float32)
    v[1, :group] = 0.25  # a flat group
    packed, s, b, mx, mean = O.quantize_affine_q4_rows(v, rows, cols, group)
    q = np.array([(packed[r * (cols // 8) + c // 8] >> (4 * (c % 8))) & 0xF for r in range(rows) for c in range(cols)],
                 np.int64).reshape(rows, cols)
    s2, b2 = s.reshape(rows, -1), b.reshape(rows, -1)
    vg = v.reshape(rows, cols // group, group)
    assert np.array_equal(b2, vg.min(axis=2))
    rng_ = vg.max(axis=2) - vg.min(axis=2)
    assert np.array_equal(s2, np.where(rng_ > 0, rng_ / np.float32(15), np.float32(1)))
    assert s2[1, 0] == 1.0 and np.all(q[1, :group] == 0)
    sc = np.repeat(s2, group, axis=1)
    bc = np.repeat(b2, group, axis=1)
    recon = (sc * q.astype(np.float32) + bc).astype(np.float32)
    err = np.abs(recon - v)
    cand = np.abs(sc[..., None] * np.arange(16, dtype=np.float32) + bc[..., None] - v[..., None])
    assert np.all(err <= cand.min(axis=2) + 2 * np.spacing(np.abs(v) + sc))  # q minimises the error
    assert mx == float(err.max())
    assert abs(mean - float(err.astype(np.float64).mean())) <= 1e-12


def test_quantizer_exact_grid_and_half_away():
    rng = np.random.default_rng(3)
    qt = rng.integers(0, 16, (4, 64))
    qt[:, 0], qt[:, 1] = 0, 15  # min and max on the grid
    v = (np.float32(-1.0) + np.float32(0.125) * qt.astype(np.float32)).astype(np.float32)
    packed, s, b, mx, _ = O.quantize_affine_q4_rows(v, 4, 64, 64)
    q = np.array([(packed[r * 8 + c // 8] >> (4 * (c % 8))) & 0xF for r in range(4) for c in range(64)]).reshape(4, 64)
    assert np.array_equal(q, qt) and mx == 0.0 and np.all(s == 0.125) and np.all(b == -1.0)
    # Range 15 -> scale 1: x.5 rounds away from zero.
    v = np.array([0.0, 15.0, 2.5, 0.5, 7.5, 14.5, 1.0, 3.0], np.float32)
    packed, _, _, _, _ = O.quantize_affine_q4_rows(v, 1, 8, 8)
    assert [(int(packed[0]) >> (4 * i)) & 0xF for i in range(8)] == [0, 15, 3, 1, 8, 15, 1, 3]


def test_quantizer_rejections():
    v = np.zeros(64, np.float32)
    for rows, cols, group in [(0, 64, 64), (1, 60, 4), (1, 64, 0), (1, 64, 48), (2, 64, 64)]:
        with pytest.raises(O.OracleError) as e:
            O.quantize_affine_q4_rows(v, rows, cols, group)
        assert e.value.code == 1
    bad = v.copy()
    bad[7] = np.inf
    with pytest.raises(O.OracleError) as e:
        O.quantize_affine_q4_rows(bad, 1, 64, 64)
    assert e.value.code == 2
