"""Single operators on the device against the oracle: nibble unpack and
dequant bit-exact; GEMV, SwiGLU, RMSNorm within the reference's tolerances
(tests/vulkan_q4_gemv_test.cpp 5e-4, vulkan_swiglu_test 2e-5,
vulkan_rmsnorm_test 3e-5) and 1e-3 relative L2 at the model's shapes."""

import numpy as np
import pytest

import oracle as O
import osm_hip
from helpers import gemv_fixture, max_abs, meta_decode, pack_q4, rel_l2, unpack_q4

pytestmark = pytest.mark.gpu


def test_unpack_nibbles_exhaustive(ctx):
    # Every value 0..15 in every lane position, plus random words: bit-exact.
    words = []
    for v in range(16):
        for lane in range(8):
            words.append(v << (4 * lane))
    rng = np.random.default_rng(0)
    words = np.concatenate([np.array(words, np.uint32), rng.integers(0, 2**32, 4096, dtype=np.uint64).astype(np.uint32)])
    out = osm_hip.unpack_nibbles(ctx, words)
    assert np.array_equal(out.reshape(-1, 8), unpack_q4(words.reshape(-1, 1)).reshape(-1, 8))


@pytest.mark.parametrize("rows,packed_cols,group", [(2, 16, 64), (37, 64, 64), (5, 8, 8), (3, 4, 4), (512, 256, 64)])
def test_dequant_bit_exact(ctx, rows, packed_cols, group):
    rng = np.random.default_rng(rows * 31 + group)
    packed = rng.integers(0, 2**32, (rows, packed_cols), dtype=np.uint64).astype(np.uint32)
    g = packed_cols * 8 // group
    s = rng.normal(0, 0.05, (rows, g)).astype(np.float32)
    b = rng.normal(0, 0.3, (rows, g)).astype(np.float32)
    gpu = osm_hip.run_q4_dequant(ctx, packed, rows, packed_cols, s, b, group)
    ora = O.dequantize_affine_rows(packed, rows, packed_cols, s, b, 4, group)
    assert np.array_equal(gpu, ora)


def test_gemv_reference_fixture(ctx):
    packed, out_dim, packed_cols, s, b, group, x = gemv_fixture()
    gpu = osm_hip.run_q4_gemv(ctx, packed, out_dim, packed_cols, s, b, group, x)
    ora = O.q4_gemv(packed, out_dim, packed_cols, s, b, group, x)
    assert max_abs(gpu, ora) <= 5e-4
    assert abs(ora[0] - ora[-1]) > 1e-3  # non-trivial rows, as the reference asserts


def test_gemv_rejects_bad_group(ctx):
    # tests/vulkan_q4_gemv_test.cpp:39-59: in_dim 8 is not divisible by group 3.
    with pytest.raises(osm_hip.OsmError) as e:
        osm_hip.run_q4_gemv(ctx, [0], 1, 1, [1.0], [0.0], 3, np.ones(8, np.float32))
    assert e.value.diagnostic


@pytest.mark.parametrize("out_dim,in_dim,group", [(512, 2048, 64), (2048, 512, 64), (96, 256, 32), (64, 256, 128), (9, 64, 8), (5, 32, 4)])
def test_gemv_shapes(ctx, out_dim, in_dim, group):
    rng = np.random.default_rng(out_dim + in_dim + group)
    q = rng.integers(0, 16, (out_dim, in_dim), dtype=np.uint32)
    s = np.abs(rng.normal(0, 0.02, (out_dim, in_dim // group))).astype(np.float32)
    b = (-8 * s + rng.normal(0, 0.002, s.shape)).astype(np.float32)
    x = rng.normal(0, 1, in_dim).astype(np.float32)
    packed = pack_q4(q)
    gpu = osm_hip.run_q4_gemv(ctx, packed, out_dim, in_dim // 8, s, b, group, x)
    ora = O.q4_gemv(packed, out_dim, in_dim // 8, s, b, group, x)
    assert rel_l2(gpu, ora) <= 1e-3
    assert max_abs(gpu, ora) <= 5e-4 * max(1.0, float(np.max(np.abs(ora))))


@pytest.mark.parametrize("meta", [osm_hip.F32, osm_hip.F16, osm_hip.BF16])
def test_gemv_preloaded_metadata_dtypes(ctx, meta):
    rng = np.random.default_rng(10 + meta)
    out_dim, in_dim, group = 512, 2048, 64
    q = rng.integers(0, 16, (out_dim, in_dim), dtype=np.uint32)
    s = meta_decode(np.abs(rng.normal(0, 0.02, (out_dim, in_dim // group))), meta)
    b = meta_decode(-8 * s + rng.normal(0, 0.002, s.shape), meta)
    x = rng.normal(0, 1, in_dim).astype(np.float32)
    packed = pack_q4(q)
    if meta == osm_hip.F32:
        sm, bm = s, b
    elif meta == osm_hip.F16:
        sm, bm = s.astype(np.float16), b.astype(np.float16)
    else:
        sm, bm = (s.view(np.uint32) >> 16).astype(np.uint16), (b.view(np.uint32) >> 16).astype(np.uint16)
    w = osm_hip.Q4ProjectionWeights(ctx, packed, out_dim, in_dim // 8, sm, bm, group, meta)
    xb, yb = osm_hip.FloatBuffer(ctx, in_dim), osm_hip.FloatBuffer(ctx, out_dim)
    xb.upload(x)
    osm_hip.run_q4_gemv_preloaded(ctx, w, xb, yb)
    gpu = yb.download()
    ora = O.q4_gemv(packed, out_dim, in_dim // 8, s, b, group, x)
    assert rel_l2(gpu, ora) <= 1e-3


def test_gemv_buffers_and_shape_checks(ctx):
    packed, out_dim, packed_cols, s, b, group, x = gemv_fixture()
    xb, yb = osm_hip.FloatBuffer(ctx, packed_cols * 8), osm_hip.FloatBuffer(ctx, out_dim)
    xb.upload(x)
    osm_hip.run_q4_gemv_buffers(ctx, packed, out_dim, packed_cols, s, b, group, xb, yb)
    assert max_abs(yb.download(), O.q4_gemv(packed, out_dim, packed_cols, s, b, group, x)) <= 5e-4
    wrong = osm_hip.FloatBuffer(ctx, out_dim + 1)
    with pytest.raises(osm_hip.OsmError):
        osm_hip.run_q4_gemv_buffers(ctx, packed, out_dim, packed_cols, s, b, group, xb, wrong)


def test_swiglu(ctx):
    rng = np.random.default_rng(3)
    g = rng.normal(0, 4, 257).astype(np.float32)
    u = rng.normal(0, 4, 257).astype(np.float32)
    gpu = osm_hip.run_swiglu(ctx, g, u)
    assert max_abs(gpu, O.swiglu(g, u)) <= 2e-5 * max(1.0, float(np.max(np.abs(gpu))))
    gb, ub, ob = (osm_hip.FloatBuffer(ctx, 257) for _ in range(3))
    gb.upload(g), ub.upload(u)
    osm_hip.run_swiglu_buffers(ctx, gb, ub, ob)
    assert np.array_equal(ob.download(), gpu)
    with pytest.raises(osm_hip.OsmError):
        osm_hip.run_swiglu(ctx, g, u[:-1])


def test_weighted_accumulate_bit_exact(ctx):
    rng = np.random.default_rng(4)
    src = rng.normal(0, 1, 257).astype(np.float32)
    acc = rng.normal(0, 1, 257).astype(np.float32)
    w = np.float32(0.3173)
    sb, ab = osm_hip.FloatBuffer(ctx, 257), osm_hip.FloatBuffer(ctx, 257)
    sb.upload(src), ab.upload(acc)
    osm_hip.run_weighted_accumulate(ctx, sb, float(w), ab)
    expect = (acc + (w * src).astype(np.float32)).astype(np.float32)
    assert np.array_equal(ab.download(), expect)
    with pytest.raises(osm_hip.OsmError):
        osm_hip.run_weighted_accumulate(ctx, sb, float("nan"), ab)


def test_rms_norm(ctx):
    rng = np.random.default_rng(5)
    v = rng.normal(0, 2, 3 * 257).astype(np.float32)
    w = (1 + rng.normal(0, 0.02, 257)).astype(np.float32)
    gpu = osm_hip.run_rms_norm(ctx, v, 3, 257, w, 1e-6)
    assert max_abs(gpu, O.rms_norm(v, 3, 257, w, 1e-6)) <= 3e-5
    with pytest.raises(osm_hip.OsmError):
        osm_hip.run_rms_norm(ctx, v, 3, 257, w[:-1], 1e-6)


# ---- affine q4 quantizer (single_expert_pilot.cpp:276-358) -------------------------------
@pytest.mark.parametrize("rows,cols,group", [(2, 8, 4), (7, 64, 8), (512, 2048, 64), (2048, 512, 64),
                                             (33, 256, 128), (5, 96, 32)])
def test_quantizer_bit_exact(ctx, rows, cols, group):
    rng = np.random.default_rng(rows * 131 + cols + group)
    if (rows, cols) == (2, 8):  # tests/affine_q4_quantizer_test.cpp:21-52
        v = np.array([-1.0, -0.5, 0.0, 0.5, 1.0, 1.5, 2.0, 2.5, 3.0, 3.0, 3.0, 3.0, -2.0, -1.0, 0.0, 1.0],
                     np.float32).reshape(2, 8)
    else:
        v = rng.normal(0, 0.05, (rows, cols)).astype(np.float32)
        v[0, :group] = -0.75  # a flat group
        v[-1, -group:] = np.round(v[-1, -group:] * 64) / 64  # values with exact half-way ratios
    gpu = osm_hip.q4_quantize(ctx, v, group)
    ora = O.quantize_affine_q4_rows(v, rows, cols, group)
    for a, b in zip(gpu[:3], ora[:3]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert gpu[3] == ora[3]
    assert abs(gpu[4] - ora[4]) <= 1e-12 * max(ora[4], 1e-30)
    # Round trip through the device dequant stays within the group bound.
    d = osm_hip.run_q4_dequant(ctx, gpu[0], rows, cols // 8, gpu[1], gpu[2], group)
    assert float(np.max(np.abs(d.reshape(rows, cols) - v))) == gpu[3]


def test_quantizer_rejections(ctx):
    v = np.zeros((2, 64), np.float32)
    with pytest.raises(osm_hip.OsmError) as e:
        osm_hip.q4_quantize(ctx, v, 48)
    assert e.value.status == osm_hip.OSM_E_INVALID
    with pytest.raises(osm_hip.OsmError) as e:
        osm_hip.q4_quantize(ctx, np.zeros((2, 60), np.float32), 4)
    assert e.value.status == osm_hip.OSM_E_INVALID
    v[1, 5] = np.nan
    with pytest.raises(osm_hip.OsmError) as e:
        osm_hip.q4_quantize(ctx, v, 64)
    assert e.value.status == osm_hip.OSM_E_RUNTIME
