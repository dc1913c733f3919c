"""The qpack container (container/qpack.cpp:41-308) and QpackExpertStorage
(storage/qpack_expert_storage.cpp:8-33): manifest.json and layout.json
parsed, every check of QpackReader::validate_container, fixed-stride reads
and their bounds, and the storage adapter -- whole slots as the reference
reads them, or slots of any section order repacked into the blob of a
geometry. CPU only.

The first group restates tests/qpack_test.cpp: its three-expert, two-layer
fixture (expertStride 16, byte value layer_seed + expert * 16 + i) and its
cases. The malformed-layout and malformed-manifest cases follow the throw
sites of parse_layout / parse_manifest / validate_container, each checked for
the reference's message."""

import json
import os

import numpy as np
import pytest

import oracle as O
import osm_hip
from helpers import blob_to_slot, qpack_q4_sections, write_qpack
from osm_hip import OSM_E_INVALID, OSM_E_RUNTIME

FIXTURE_SECTIONS = [
    {"name": "gate_proj.weight", "dtype": "U32", "shape": (2, 2), "offset": 0, "size": 8},
    {"name": "gate_proj.scales", "dtype": "BF16", "shape": (2,), "offset": 8, "size": 4},
]


def fixture_slots(seed):
    """tests/qpack_test.cpp:32-46: three experts of 16 bytes, byte i of
    expert e is seed + e * 16 + i."""
    return np.array([[(seed + e * 16 + i) % 256 for i in range(16)] for e in range(3)], np.uint8)


def make_fixture(root, magic="QPACK", quant_group_size=8, **kw):
    """tests/qpack_test.cpp:48-94 (layer seeds 0 and 64; linearLayers
    [true, false]; 4-bit, group 8: 2 packed words x 8 = 2 groups x 8)."""
    return write_qpack(str(root), [fixture_slots(0), fixture_slots(64)], FIXTURE_SECTIONS, 16,
                       linear_layers=[True, False], magic=magic, quant_group_size=quant_group_size, **kw)


def open_error(root):
    with pytest.raises(osm_hip.OsmError) as ei:
        osm_hip.QpackReader(str(root))
    return ei.value


# ---- tests/qpack_test.cpp ----------------------------------------------------------

def test_parse_and_read(tmp_path):
    r = osm_hip.QpackReader(make_fixture(tmp_path))
    assert r.magic == "QPACK" and r.version == 1 and r.model_name == "qwen3_next"
    assert r.quant_bits == 4 and r.quant_group_size == 8
    assert (r.expert_count, r.layer_count, r.expert_stride) == (3, 2, 16)
    assert r.linear_layers == [True, False]
    s = r.find_section("gate_proj.weight")
    assert s is not None and s["offset"] == 0 and s["size"] == 8 and s["shape"] == [2, 2]
    assert r.find_section("up_proj.weight") is None
    assert r.sections[1] == {"name": "gate_proj.scales", "dtype": "BF16", "shape": [2], "offset": 8, "size": 4}
    got = r.read_expert(1, 2)
    assert got.size == 16 and np.array_equal(got, (64 + 2 * 16 + np.arange(16)).astype(np.uint8))
    assert r.file_size("packed_experts/layer_00.bin") == 48 and r.file_size("nope.bin") is None


def test_rejects_bad_magic(tmp_path):
    e = open_error(make_fixture(tmp_path, magic="NOT_QPACK"))
    assert e.status == OSM_E_RUNTIME and "unsupported magic: NOT_QPACK" in str(e)


def test_rejects_short_layer(tmp_path):
    make_fixture(tmp_path)
    os.truncate(tmp_path / "packed_experts" / "layer_01.bin", 47)
    e = open_error(tmp_path)
    assert e.status == OSM_E_RUNTIME and "expert layer has unexpected byte size" in str(e)


def test_rejects_quant_shape_mismatch(tmp_path):
    e = open_error(make_fixture(tmp_path, quant_group_size=64))
    assert "expert quantization disagrees with packed shapes: gate_proj" in str(e)


def test_storage_adapter(tmp_path):
    st = osm_hip.QpackStorage(make_fixture(tmp_path))
    assert st.stride == 16
    first, second = st.read([0, 1], [1, 2])
    assert np.array_equal(first, (16 + np.arange(16)).astype(np.uint8))
    assert np.array_equal(second, (64 + 32 + np.arange(16)).astype(np.uint8))


def test_bounds(tmp_path):
    r = osm_hip.QpackReader(make_fixture(tmp_path))
    for layer, expert, n, what in [(2, 0, 16, "layer index out of range"), (0, 3, 16, "expert index out of range"),
                                   (0, 0, 8, "destination is smaller than expertStride")]:
        with pytest.raises(osm_hip.OsmError) as ei:
            r.read_expert(layer, expert, n)
        assert ei.value.status == OSM_E_INVALID and what in str(ei.value)
    st = osm_hip.QpackStorage(str(tmp_path))
    with pytest.raises(osm_hip.OsmError) as ei:
        st.read([2], [0])
    assert ei.value.status == OSM_E_INVALID
    with pytest.raises(osm_hip.OsmError) as ei:
        st.read([0], [0], dest_bytes=15)
    assert ei.value.status == OSM_E_INVALID


# ---- malformed layouts and manifests (qpack.cpp:61-255) ----------------------------

def layout_doc(**over):
    doc = {"expertCount": 3, "layerCount": 2, "expertStride": 16,
           "sections": [dict(s, shape=list(s["shape"])) for s in FIXTURE_SECTIONS], "linearLayers": [True, False]}
    for k, v in over.items():
        if v is None:
            doc.pop(k)
        else:
            doc[k] = v
    return json.dumps(doc)


def sec(**over):
    s = dict(FIXTURE_SECTIONS[0], shape=[2, 2])
    s.update(over)
    return s


@pytest.mark.parametrize("text,message", [
    ("{not json", "invalid JSON in"),
    ('{"expertCount": 3, "expertCount": 3}', "invalid JSON in"),  # duplicate key
    (layout_doc(expertCount=None), "malformed layout"),
    (layout_doc(expertCount="3"), "malformed layout"),
    (layout_doc(expertCount=-3), "malformed layout"),
    (layout_doc(expertCount=2.5), "malformed layout"),
    (layout_doc(layerCount=2 ** 32), "malformed layout"),
    (layout_doc(expertStride=None), "malformed layout"),
    (layout_doc(linearLayers=None), "malformed layout"),
    (layout_doc(linearLayers=[1, 0]), "malformed layout"),
    (layout_doc(sections={"a": 1}), "layout.sections must be an array"),
    (layout_doc(sections=[{"dtype": "U32", "shape": [2], "offset": 0, "size": 8}]), "malformed layout"),
    (layout_doc(sections=[sec(shape=2)]), "malformed layout"),
    (layout_doc(sections=[sec(offset=-1)]), "malformed layout"),
    (layout_doc(layerCount=0, linearLayers=[]), "layerCount must be non-zero"),
    (layout_doc(sections=[]), "sections must not be empty"),
    (layout_doc(linearLayers=[True]), "linearLayers length must equal layerCount"),
    (layout_doc(sections=[sec(name="")]), "section name/size is invalid"),
    (layout_doc(sections=[sec(size=0)]), "section name/size is invalid"),
    (layout_doc(sections=[sec(offset=12, size=8)]), "section exceeds expertStride: gate_proj.weight"),
    (layout_doc(sections=[sec(offset=17, size=1)]), "section exceeds expertStride"),
    (layout_doc(expertStride=0, sections=[sec(size=1, offset=0)]), "section exceeds expertStride"),
    (layout_doc(expertCount=0), "expertCount and expertStride must be non-zero"),
    (layout_doc(expertStride=2 ** 63, expertCount=3), "layer byte size overflows uint64"),
    (layout_doc(sections=[sec(), dict(FIXTURE_SECTIONS[1], shape=[])]), "quantized expert section has empty shape"),
])
def test_malformed_layouts(tmp_path, text, message):
    make_fixture(tmp_path, layout_text=text)
    e = open_error(tmp_path)
    assert e.status == OSM_E_RUNTIME and message in str(e), str(e)


def rewrite_manifest(root, **over):
    path = os.path.join(root, "manifest.json")
    with open(path) as f:
        m = json.load(f)
    for k, v in over.items():
        if v is ...:
            m.pop(k)
        else:
            m[k] = v
    with open(path, "w") as f:
        json.dump(m, f)


@pytest.mark.parametrize("over,message", [
    (dict(magic=...), "malformed manifest"),
    (dict(version="1"), "malformed manifest"),
    (dict(version=2), "unsupported manifest version: 2"),
    (dict(modelName=7), "malformed manifest"),
    (dict(files=[]), "manifest.files must be an object"),
    (dict(files={"packed_experts/layout.json": -1}), "malformed manifest"),
    (dict(quantGroupSize=None), "quantBits and quantGroupSize must both be present or both be null"),
    (dict(quantBits=3), "invalid expert quantization metadata"),
    (dict(quantBits=0), "invalid expert quantization metadata"),
])
def test_malformed_manifests(tmp_path, over, message):
    make_fixture(tmp_path)
    rewrite_manifest(str(tmp_path), **over)
    e = open_error(tmp_path)
    assert e.status == OSM_E_RUNTIME and message in str(e), str(e)


def test_null_quantization_skips_the_shape_check(tmp_path):
    # quantBits / quantGroupSize both null: no quantization check at all
    # (qpack.cpp:136-142), so the group-64 mismatch passes.
    make_fixture(tmp_path)
    rewrite_manifest(str(tmp_path), quantBits=None, quantGroupSize=None)
    r = osm_hip.QpackReader(str(tmp_path))
    assert r.quant_bits is None and r.quant_group_size is None
    rewrite_manifest(str(tmp_path), quantBits=..., quantGroupSize=...)  # absent keys read as null
    assert osm_hip.QpackReader(str(tmp_path)).quant_bits is None


def test_declared_files(tmp_path):
    make_fixture(tmp_path, declare=False)
    e = open_error(tmp_path)
    assert "manifest does not declare required file: packed_experts/layer_00.bin" in str(e)
    make_fixture(tmp_path)
    with open(tmp_path / "manifest.json") as f:
        m = json.load(f)
    m["files"]["packed_experts/layout.json"] += 1
    with open(tmp_path / "manifest.json", "w") as f:
        json.dump(m, f)
    assert "file size disagrees with manifest: packed_experts/layout.json" in str(open_error(tmp_path))
    make_fixture(tmp_path)
    os.remove(tmp_path / "packed_experts" / "layer_01.bin")
    assert "missing expert layer file" in str(open_error(tmp_path))
    os.remove(tmp_path / "manifest.json")
    assert "unable to open JSON file" in str(open_error(tmp_path))


def test_json_text_forms(tmp_path):
    # Whitespace, escapes, a \u pair in a string, exponent-written whole
    # numbers and unknown keys are all accepted; trailing text is not.
    doc = json.loads(layout_doc())
    doc["commenté"] = "😀 \"quoted\" \\ / \t"
    doc["nested"] = {"a": [1, 2, {"b": None}], "c": False}
    text = json.dumps(doc, ensure_ascii=True).replace('"expertStride": 16', '"expertStride": 1.6e1')
    make_fixture(tmp_path, layout_text=text)
    assert osm_hip.QpackReader(str(tmp_path)).expert_stride == 16
    make_fixture(tmp_path, layout_text=layout_doc() + " x")
    assert "invalid JSON in" in str(open_error(tmp_path))
    make_fixture(tmp_path, layout_text="[" * 100 + "]" * 100)
    assert "invalid JSON in" in str(open_error(tmp_path))


# ---- slots of any section order, repacked into the blob ----------------------------

@pytest.mark.parametrize("meta,dt", [(O.META_BF16, "BF16"), (O.META_F32, "F32")])
def test_storage_repacks_noncanonical_slots(tmp_path, meta, dt):
    D, I, G, E, L = 256, 128, 64, 5, 2
    g = osm_hip.geometry(D, I, G, meta)
    order = ["down_proj.weight", "up_proj.biases", "gate_proj.scales", "up_proj.weight", "down_proj.scales",
             "gate_proj.weight", "gate_proj.biases", "up_proj.scales", "down_proj.biases"]
    secs, stride = qpack_q4_sections(D, I, G, dt, order=order, gap=24,
                                     extra=[("router_hint.bias", "F32", (7,), 28)])
    blobs = [[O.synth_expert_blob(3, l, e, D, I, G, meta=meta) for e in range(E)] for l in range(L)]
    slots = [np.stack([blob_to_slot(b, secs, stride, D, I, G, dt) for b in layer]) for layer in blobs]
    write_qpack(str(tmp_path), slots, secs, stride, quant_group_size=G)
    raw = osm_hip.QpackStorage(str(tmp_path))
    assert raw.stride == stride
    st = osm_hip.QpackStorage(str(tmp_path), g)
    assert st.stride == osm_hip.expert_blob_bytes(g) < stride
    ls, es = [1, 0, 1, 0, 1], [4, 0, 2, 3, 0]
    for l, e, got in zip(ls, es, st.read(ls, es)):
        assert np.array_equal(got, blobs[l][e]), (l, e)
    for l, e, got in zip(ls, es, raw.read(ls, es)):
        assert np.array_equal(got, slots[l][e])
    # The host L1 cache over it holds blobs.
    host = osm_hip.HostExpertCache.from_storage(st, 3 * st.stride)
    _, got = host.fetch(1, [2, 4])
    assert np.array_equal(got[0], blobs[1][2]) and np.array_equal(got[1], blobs[1][4])


def test_official_layout_reads_straight_through(tmp_path):
    D, I, G, E = 256, 128, 64, 3
    g = osm_hip.geometry(D, I, G, O.META_BF16)
    secs, stride = qpack_q4_sections(D, I, G, "BF16")
    blobs = [O.synth_expert_blob(4, 0, e, D, I, G) for e in range(E)]
    write_qpack(str(tmp_path), [np.stack(blobs)], secs, stride, quant_group_size=G)
    st = osm_hip.QpackStorage(str(tmp_path), g)
    assert st.stride == stride
    for e, got in enumerate(st.read([0] * E, list(range(E)))):
        assert np.array_equal(got, blobs[e])


def test_storage_rejects_tables_the_geometry_cannot_bind(tmp_path):
    D, I, G = 256, 128, 64
    secs, stride = qpack_q4_sections(D, I, G, "BF16")
    write_qpack(str(tmp_path), [np.zeros((2, stride), np.uint8)], secs, stride, quant_group_size=G)
    with pytest.raises(osm_hip.OsmError) as ei:  # wider hidden than the table
        osm_hip.QpackStorage(str(tmp_path), osm_hip.geometry(512, I, G, O.META_BF16))
    assert ei.value.status == OSM_E_RUNTIME
    with pytest.raises(osm_hip.OsmError) as ei:  # F32 metadata asked of BF16 sections
        osm_hip.QpackStorage(str(tmp_path), osm_hip.geometry(D, I, G, O.META_F32))
    assert ei.value.status == OSM_E_INVALID
    drop = [s for s in secs if s["name"] != "up_proj.biases"]
    write_qpack(str(tmp_path), [np.zeros((2, stride), np.uint8)], drop, stride, quant_group_size=G)
    with pytest.raises(osm_hip.OsmError) as ei:
        osm_hip.QpackStorage(str(tmp_path), osm_hip.geometry(D, I, G, O.META_BF16))
    assert "section set is incomplete" in str(ei.value)
