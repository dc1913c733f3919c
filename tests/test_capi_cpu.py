"""libosm_hip.so without a device: it loads, exports every entry point that
include/osm_hip.h declares, lays out expert blobs as documented, and fails
with a diagnostic (never a silent fallback) when no HIP device is present."""

import os
import re
import subprocess

import numpy as np
import pytest

import oracle as O
import osm_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "osm_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(osm_[a-z0-9_]+)\s*\(", text))
    names.discard("osm_read_experts_fn")
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = osm_hip.load()
    names = declared_functions()
    assert len(names) > 60
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # The binding covers exactly the header.
    assert sorted(osm_hip.exported_symbols()) == names
    out = subprocess.run(["nm", "-D", "--defined-only", osm_hip.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (osm_[a-z0-9_]+)", out))
    assert set(names) <= exported


def test_blob_layout_sizes():
    # One expert of the Qwen3-Next geometry (2048/512/group 64): 1,769,472 B with
    # bf16 metadata; 1,966,080 B with f32 metadata (the reference converter's
    # expertStride, docs/OSM-39B-QPACK-EXPERT-GEOMETRY.md:61-74).
    assert osm_hip.expert_blob_bytes(osm_hip.geometry(2048, 512, 64, osm_hip.BF16)) == 1769472
    assert osm_hip.expert_blob_bytes(osm_hip.geometry(2048, 512, 64, osm_hip.F32)) == 1966080
    assert osm_hip.expert_blob_bytes(osm_hip.geometry(128, 64, 64, osm_hip.BF16)) == 13824
    for g in [(2048, 512, 64, 2), (128, 64, 64, 0), (256, 96, 32, 1)]:
        assert osm_hip.expert_blob_bytes(osm_hip.geometry(*g)) == O.expert_blob_bytes(*g)
    # Unsupported by the fused kernels -> 0.
    assert osm_hip.expert_blob_bytes(osm_hip.geometry(100, 64, 64, 2)) == 0
    assert osm_hip.expert_blob_bytes(osm_hip.geometry(128, 64, 48, 2)) == 0


def test_no_device_fails_loudly():
    if osm_hip.device_count() > 0:
        pytest.skip("a HIP device is present")
    with pytest.raises(osm_hip.OsmError) as e:
        osm_hip.Context(0)
    assert e.value.status == osm_hip.OSM_E_DEVICE and e.value.diagnostic


def test_generator_statistics_and_determinism():
    n = 200000
    stream = O.lib().oracle_synth_stream(1234, 0, 7, 1)
    v = np.array([O.lib().oracle_synth_normal(stream, i) for i in range(0, n, 4)], np.float64)
    assert abs(v.mean()) < 0.02 and abs(v.std() - 1.0) < 0.02
    # Irwin-Hall(12): support [-6, 6], excess kurtosis -0.1, and N(0,1)'s
    # tail mass beyond 3 sigma (0.27%: 135 of 50,000 expected).
    assert np.max(np.abs(v)) <= 6.0
    assert abs(np.mean(v ** 4) - 2.9) < 0.1
    assert 90 < np.count_nonzero(np.abs(v) > 3.0) < 190
    # The integer sum is exact and the scale a power of two, so every draw is
    # a multiple of 2^-16 and the extremes are reachable.
    assert np.all(v * 65536.0 == np.round(v * 65536.0))
    blob = O.synth_expert_blob(5, 1, 2, 2048, 512)
    again = O.synth_expert_blob(5, 1, 2, 2048, 512)
    other = O.synth_expert_blob(5, 1, 3, 2048, 512)
    assert np.array_equal(blob, again) and not np.array_equal(blob, other)
    secs = O.blob_sections(blob, 2048, 512)
    from helpers import unpack_q4
    q = unpack_q4(secs[0][0])
    counts = np.bincount(q.ravel(), minlength=16)
    assert counts.min() > 0.9 * q.size / 16 and counts.max() < 1.1 * q.size / 16
    s_, b_ = secs[0][1], secs[0][2]
    assert np.all(s_ >= 0) and abs(np.mean(s_) - 0.02 * np.sqrt(2 / np.pi)) < 0.002
    assert abs(np.mean(b_ + 8 * s_)) < 0.001 and abs(np.std(b_ + 8 * s_) - 0.002) < 0.0005


def test_argument_checks_before_any_device_work():
    # Entry points that reject their arguments before touching a device: the
    # native cached layer stack, the qpack binding and the pread storage.
    import ctypes
    lib = osm_hip.load()
    st = lib.osm_moe_run_cached_layers(None, None, None, 0, None, None, 0, None, None, None)
    assert st == osm_hip.OSM_E_INVALID and osm_hip.last_error()
    g = osm_hip.geometry(256, 128, 64, osm_hip.BF16)
    assert lib.osm_qpack_expert_repack(ctypes.byref(g), None, 3, 0, None, None, 0, None) == osm_hip.OSM_E_INVALID
    h = ctypes.c_void_p()
    assert lib.osm_pread_storage_create(None, 1, 1, 16, ctypes.byref(h)) == osm_hip.OSM_E_INVALID
    assert lib.osm_pread_storage_create(b"/nonexistent", 0, 1, 16, ctypes.byref(h)) == osm_hip.OSM_E_INVALID
    assert lib.osm_expert_storage_stride(None) == 0
    assert lib.osm_host_cache_create_with_storage(None, 1 << 20, 1, 0, ctypes.byref(h)) == osm_hip.OSM_E_INVALID
