"""Expert blobs read from a container directory with pread
(storage/posix_pread_expert_storage.cpp:98-187), alone and as the host L1
cache's storage (cache/expert_cache.cpp:101-200). CPU only: the cache's slots
are pageable here."""

import os

import numpy as np
import pytest

import osm_hip
from osm_hip import OSM_E_INVALID, OSM_E_RUNTIME


def write_container(root, layers, experts, stride, seed, short_layer=None):
    rng = np.random.default_rng(seed)
    blobs = rng.integers(0, 256, (layers, experts, stride), dtype=np.uint8)
    os.makedirs(os.path.join(root, "packed_experts"), exist_ok=True)
    for l in range(layers):
        data = blobs[l].reshape(-1)
        if l == short_layer:
            data = data[: -(stride // 2)]  # the last expert is cut in half
        data.tofile(osm_hip.PreadStorage.layer_path(root, l))
    return blobs


def test_reads_every_requested_blob(tmp_path):
    # An odd stride (no alignment assumed), 40 requests in one call (read in
    # parallel), repeats and both layers mixed.
    layers, experts, stride = 2, 7, 1000 + 13
    blobs = write_container(str(tmp_path), layers, experts, stride, 1)
    st = osm_hip.PreadStorage(str(tmp_path), layers, experts, stride)
    assert osm_hip.load().osm_expert_storage_stride(st.h) == stride
    rng = np.random.default_rng(2)
    ls = rng.integers(0, layers, 40)
    es = rng.integers(0, experts, 40)
    got = st.read(ls, es)
    for l, e, g in zip(ls, es, got):
        assert np.array_equal(g, blobs[l, e])
    # a destination larger than the stride: the rest is left alone
    big = st.read([1], [6], dest_bytes=stride + 64)[0]
    assert np.array_equal(big[:stride], blobs[1, 6])


def test_request_errors(tmp_path):
    layers, experts, stride = 2, 4, 512
    write_container(str(tmp_path), layers, experts, stride, 3, short_layer=1)
    st = osm_hip.PreadStorage(str(tmp_path), layers, experts, stride)
    for ls, es in (([2], [0]), ([0], [4])):  # layer, expert out of range
        with pytest.raises(osm_hip.OsmError) as e:
            st.read(ls, es)
        assert e.value.status == OSM_E_INVALID
    with pytest.raises(osm_hip.OsmError) as e:
        st.read([0], [0], dest_bytes=stride - 1)
    assert e.value.status == OSM_E_INVALID
    with pytest.raises(osm_hip.OsmError) as e:  # the cut expert: a short read
        st.read([0, 1], [3, 3])
    assert e.value.status == OSM_E_RUNTIME and "short" in str(e.value)
    assert st.read([1], [2])[0].size == stride  # the rest of that layer reads
    missing = osm_hip.PreadStorage(str(tmp_path / "absent"), layers, experts, stride)
    with pytest.raises(osm_hip.OsmError) as e:
        missing.read([0], [0])
    assert e.value.status == OSM_E_RUNTIME
    with pytest.raises(osm_hip.OsmError) as e:
        osm_hip.PreadStorage(str(tmp_path), layers, experts, 0)
    assert e.value.status == OSM_E_INVALID


def test_host_cache_over_pread_storage(tmp_path):
    # Three slots: the fetches of the reference's cache test pattern, with the
    # bytes served from the files.
    layers, experts, stride = 1, 6, 2048
    blobs = write_container(str(tmp_path), layers, experts, stride, 4)
    st = osm_hip.PreadStorage(str(tmp_path), layers, experts, stride)
    cache = osm_hip.HostExpertCache.from_storage(st, 3 * stride)
    slots, got = cache.fetch(0, [0, 1, 2])
    for e, g in zip((0, 1, 2), got):
        assert np.array_equal(g, blobs[0, e])
    assert cache.stats()["misses"] == 3 and cache.stats()["hits"] == 0
    _, got = cache.fetch(0, [1, 4])  # 1 hits; 4 evicts the least used
    assert np.array_equal(got[0], blobs[0, 1]) and np.array_equal(got[1], blobs[0, 4])
    st_ = cache.stats()
    assert (st_["hits"], st_["misses"]) == (1, 4)
    assert cache.resident_slot(0, 4) is not None
    with pytest.raises(osm_hip.OsmError):
        cache.fetch(0, [5, 6])  # expert 6 is out of range: nothing is cached
    assert cache.resident_slot(0, 5) is None
