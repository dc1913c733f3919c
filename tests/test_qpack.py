"""An expert's qpack cache slot bound by section name
(backend/vulkan_qpack_expert.cpp:149-239): the official contiguous layout
(docs/OSM-39B-QPACK-EXPERT-GEOMETRY.md:35-42) is the blob as it stands, any
other order and spacing is repacked section by section, and every check of
the reference's binding rejects what it rejects. CPU only."""

import numpy as np
import pytest

import oracle as O
import osm_hip
from osm_hip import OSM_E_INVALID, OSM_E_RUNTIME

PROJ = ("gate_proj", "up_proj", "down_proj")


def sections_for(D, I, G, meta_dtype, order=None, gap=0):
    """Section table of one slot: the nine sections in `order` (names), each
    followed by `gap` bytes."""
    esz = 4 if meta_dtype == "F32" else 2
    shapes = {}
    for p in PROJ:
        out, inn = (I, D) if p != "down_proj" else (D, I)
        shapes[p + ".weight"] = ("U32", (out, inn // 8), out * inn // 8 * 4)
        shapes[p + ".scales"] = (meta_dtype, (out, inn // G), out * inn // G * esz)
        shapes[p + ".biases"] = (meta_dtype, (out, inn // G), out * inn // G * esz)
    names = order or [p + s for p in PROJ for s in (".weight", ".scales", ".biases")]
    secs, off = [], 0
    for n in names:
        dt, shape, size = shapes[n]
        secs.append({"name": n, "dtype": dt, "shape": shape, "offset": off, "size": size})
        off += size + gap
    return secs, off


def canonical_parts(blob, D, I, G, meta):
    """The blob's nine sections by name (canonical order)."""
    esz = 4 if meta == O.META_F32 else 2
    parts, off = {}, 0
    for p in PROJ:
        out, inn = (I, D) if p != "down_proj" else (D, I)
        for s, n in ((".weight", out * inn // 2), (".scales", out * inn // G * esz), (".biases", out * inn // G * esz)):
            parts[p + s] = blob[off:off + n]
            off += n
    return parts


@pytest.mark.parametrize("meta,dt", [(O.META_F32, "F32"), (O.META_BF16, "BF16")])
def test_official_layout_is_the_blob(meta, dt):
    D, I, G = 256, 128, 64
    g = osm_hip.geometry(D, I, G, meta)
    blob = O.synth_expert_blob(5, 0, 3, D, I, G, meta=meta)
    secs, stride = sections_for(D, I, G, dt)
    assert stride == blob.size
    got, ident = osm_hip.qpack_expert_repack(g, secs, stride, blob)
    assert ident and np.array_equal(got, blob)


def test_other_orders_are_repacked():
    D, I, G = 256, 128, 32
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    blob = O.synth_expert_blob(6, 0, 1, D, I, G, meta=O.META_BF16)
    parts = canonical_parts(blob, D, I, G, O.META_BF16)
    order = ["down_proj.biases", "up_proj.weight", "gate_proj.scales", "down_proj.weight", "gate_proj.weight",
             "up_proj.biases", "gate_proj.biases", "down_proj.scales", "up_proj.scales"]
    secs, used = sections_for(D, I, G, "BF16", order=order, gap=64)
    stride = used + 4096  # slack at the end of the slot, as a padded stride would leave
    slot = np.random.default_rng(0).integers(0, 256, stride, dtype=np.uint8)
    for s in secs:
        slot[s["offset"]:s["offset"] + s["size"]] = parts[s["name"]]
    got, ident = osm_hip.qpack_expert_repack(g, secs, stride, slot)
    assert not ident and np.array_equal(got, blob)
    _, ident = osm_hip.qpack_expert_repack(g, secs, stride)  # validation alone
    assert not ident


def test_rejected_tables():
    D, I, G = 256, 128, 64
    g = osm_hip.geometry(D, I, G, osm_hip.F32)
    good, stride = sections_for(D, I, G, "F32")

    def bad(mutate, status=OSM_E_RUNTIME, stride_=stride):
        secs = [dict(s) for s in good]
        mutate(secs)
        with pytest.raises(osm_hip.OsmError) as e:
            osm_hip.qpack_expert_repack(g, secs, stride_)
        assert e.value.status == status, e.value.diagnostic

    bad(lambda s: s.pop(4))                                       # up_proj.scales missing
    bad(lambda s: s[0].update(dtype="F32"))                       # weight must be U32
    bad(lambda s: s[2].update(dtype="F16"))                       # scales/biases differ
    bad(lambda s: [x.update(dtype="F8") for x in s[1:3]])         # unsupported metadata dtype
    bad(lambda s: [x.update(dtype="BF16", size=x["size"] // 2) for x in s if x["dtype"] == "F32"],
        OSM_E_INVALID)                                            # not the geometry's dtype
    bad(lambda s: s[6].update(shape=(I, D // 8)))                 # down weight with gate's shape
    bad(lambda s: s[3].update(size=s[3]["size"] - 4))             # size disagrees with shape
    bad(lambda s: s[8].update(offset=s[8]["offset"] + 2))         # misaligned (and past the end)
    bad(lambda s: None, stride_=stride - 4)                       # last section past the slot
    secs = [dict(s) for s in good]
    secs[0]["shape"] = (I,)  # rank 1
    with pytest.raises(osm_hip.OsmError):
        osm_hip.qpack_expert_repack(g, secs, stride)
