"""Cache policies, host-only: the oracle restatement pinned by the reference's
own scenarios (tests/expert_cache_test.cpp, tests/vulkan_resident_expert_cache_test.cpp)
and by the reference's ExpertCache compiled into oracle/_ref, then the
product's policies (through the C ABI, no device needed) against the oracle
on random access traces -- exact counters, slots and victims."""

import numpy as np
import pytest

import oracle as O
import osm_hip

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference checkout)")


def _pattern(layer, expert, stride):
    return ((layer * 37 + expert * 11 + np.arange(stride)) & 0xFF).astype(np.uint8)


# ---- host L1 cache: the reference test's scenarios (expert_cache_test.cpp:78-193) -----------
@pytest.mark.parametrize("impl", ["oracle", pytest.param("ref", marks=needs_ref)])
def test_host_cache_reference_scenarios(impl):
    c = O.HostCache(8, 8 * 3, impl=impl)
    slots, ok = c.fetch(0, [1, 2])
    assert ok and len(slots) == 2
    st = c.stats()
    assert (st["hits"], st["misses"], st["allocated_slots"]) == (0, 2, 2) and c.storage_batches() == 1
    slots2, ok = c.fetch(0, [2, 1])
    assert ok and slots2 == slots[::-1]
    st = c.stats()
    assert (st["hits"], st["misses"]) == (2, 2) and c.storage_batches() == 1

    c = O.HostCache(4, 8, impl=impl)
    for e in (0, 0, 1, 2):
        c.fetch(0, [e])
    assert c.resident_slot(0, 0) is not None and c.resident_slot(0, 1) is None and c.resident_slot(0, 2) is not None
    c = O.HostCache(4, 8, impl=impl)
    for e in (0, 1, 2):
        c.fetch(0, [e])
    assert c.resident_slot(0, 0) is None and c.resident_slot(0, 1) is not None

    c = O.HostCache(8, 16, impl=impl)
    c.fetch(0, [0, 1])
    s, _ = c.fetch(0, [2, 3])
    assert s[0] != s[1] and c.resident_slot(0, 2) is not None and c.resident_slot(0, 3) is not None

    c = O.HostCache(8, 24, impl=impl)
    c.fetch(1, [0])
    stable = c.resident_slot(1, 0)
    with pytest.raises(O.OracleError):
        c.fetch(1, [1, 2], fail_read=True)
    assert c.resident_slot(1, 0) == stable and c.resident_slot(1, 1) is None and c.resident_slot(1, 2) is None
    assert c.stats()["allocated_slots"] == 3

    c = O.HostCache(4, 8, impl=impl)
    with pytest.raises(O.OracleError):
        c.fetch(0, [0, 1, 2])
    assert c.stats()["allocated_slots"] == 0 and c.storage_batches() == 0


def _random_trace(seed, n, layers=3, experts=9, batch_max=3):
    rng = np.random.default_rng(seed)
    trace = []
    for _ in range(n):
        layer = int(rng.integers(0, layers))
        b = int(rng.integers(1, batch_max + 1))
        trace.append((layer, [int(v) for v in rng.integers(0, experts, b)], bool(rng.random() < 0.05)))
    return trace


@needs_ref
@pytest.mark.parametrize("seed", range(4))
def test_host_cache_oracle_matches_reference_build(seed):
    a, r = O.HostCache(16, 16 * 5, impl="oracle"), O.HostCache(16, 16 * 5, impl="ref")
    for layer, batch, fail in _random_trace(seed, 300):
        try:
            sa, _ = a.fetch(layer, batch, fail_read=fail)
            ea = None
        except O.OracleError as e:
            sa, ea = None, e.code
        try:
            sr, _ = r.fetch(layer, batch, fail_read=fail)
            er = None
        except O.OracleError as e:
            sr, er = None, e.code
        assert (sa, ea) == (sr, er)
    assert a.stats() == r.stats() and a.storage_batches() == r.storage_batches()
    for layer in range(3):
        for e in range(9):
            assert a.resident_slot(layer, e) == r.resident_slot(layer, e)


# ---- resident cache policy: the reference scenario (vulkan_resident_expert_cache_test.cpp:316-382)
def test_device_policy_reference_scenario():
    acc = 17152  # the reference fixture's accounted bytes per expert
    p = O.DeviceCachePolicy(2 * acc)
    assert p.get(0, 0, acc) == (False, [])
    assert p.get(0, 1, acc) == (False, [])
    st = p.stats()
    assert (st["hits"], st["misses"], st["loads"], st["evictions"], st["resident_entries"]) == (0, 2, 2, 0, 2)
    assert p.get(0, 0, acc) == (True, [])
    hit, ev = p.get(0, 2, acc)
    assert not hit and ev == [1]  # LFU: expert 1 (frequency 1) leaves, expert 0 (frequency 2) stays
    st = p.stats()
    assert (st["hits"], st["misses"], st["loads"], st["evictions"], st["resident_entries"]) == (1, 3, 3, 1, 2)
    assert p.contains(0, 0) and not p.contains(0, 1) and p.contains(0, 2)
    # Equal frequencies: the least recently used goes first; history survives eviction.
    q = O.DeviceCachePolicy(2)
    q.get(0, 5, 1), q.get(0, 6, 1)
    assert q.get(0, 7, 1) == (False, [5])
    assert q.get(0, 5, 1) == (False, [6])  # 5 returns with frequency 2, 6 (freq 1) is evicted
    with pytest.raises(O.OracleError):
        O.DeviceCachePolicy(4).get(0, 1, 5)


def test_device_policy_batch_evicts_its_own_earlier_pick():
    # One fill batch of two tokens picking [0, 1] and [1, 0] over a 4-expert
    # budget warmed with 10-13 at frequency 2: 0 takes 10's place, 1 evicts 0
    # (this batch's own frequency-1 fill), 1 hits, and 0 comes back in 11's
    # place. Token 0's pick 0 is resident at the end, but not in the slot it
    # was first copied to, which 1 now holds: a layer that runs every pick of
    # the batch after all the gets must look its slot up again. Oracle and
    # product policy agree on every step.
    for p in (O.DeviceCachePolicy(4), osm_hip.CachePolicy(4)):
        for _ in range(2):
            for e in (10, 11, 12, 13):
                p.get(0, e, 1)
        steps = [p.get(0, e, 1) for e in (0, 1, 1, 0)]
        assert steps == [(False, [10]), (False, [0]), (True, []), (False, [11])]
        assert p.contains(0, 0) and p.contains(0, 1) and not p.contains(0, 10) and not p.contains(0, 11)


# ---- product policies through the C ABI, against the oracle --------------------------------
@pytest.mark.parametrize("seed", range(5))
def test_product_policy_matches_oracle(seed):
    rng = np.random.default_rng(seed)
    budget = 7
    a, b = osm_hip.CachePolicy(budget), O.DeviceCachePolicy(budget)
    for _ in range(2000):
        layer, expert = int(rng.integers(0, 4)), int(rng.integers(0, 12))
        nbytes = int(rng.integers(1, 3))
        assert a.get(layer, expert, nbytes) == b.get(layer, expert, nbytes)
    assert a.stats() == b.stats()


def test_product_policy_rejections():
    p = osm_hip.CachePolicy(4)
    with pytest.raises(osm_hip.OsmError) as e:
        p.get(0, 1, 5)
    assert "exceeds the configured budget" in e.value.diagnostic
    with pytest.raises(osm_hip.OsmError) as e:
        p.get(0, 1, 0)
    assert "accounting is zero" in e.value.diagnostic
    with pytest.raises(osm_hip.OsmError):
        osm_hip.CachePolicy(0)


@pytest.mark.parametrize("seed", range(4))
def test_product_host_cache_matches_oracle(seed):
    stride = 16
    fail_box = {"fail": False}

    def read(layers, experts, dests):
        if fail_box["fail"]:
            return 1
        for l, e, d in zip(layers, experts, dests):
            d[:] = _pattern(l, e, stride)
        return 0

    a = osm_hip.HostExpertCache(stride, stride * 5, read, pinned=False)
    b = O.HostCache(stride, stride * 5, impl="oracle")
    for layer, batch, fail in _random_trace(100 + seed, 300):
        fail_box["fail"] = fail
        try:
            sa, blobs = a.fetch(layer, batch)
            ea = None
            for e, bl in zip(batch, blobs):
                assert np.array_equal(bl, _pattern(layer, e, stride))
        except osm_hip.OsmError:
            sa, ea = None, "err"
        try:
            sb, _ = b.fetch(layer, batch, fail_read=fail)
            eb = None
        except O.OracleError:
            sb, eb = None, "err"
        assert (None if sa is None else [int(v) for v in sa], ea) == (sb, eb)
    assert a.stats() == b.stats()
    for layer in range(3):
        for e in range(9):
            assert a.resident_slot(layer, e) == b.resident_slot(layer, e)
