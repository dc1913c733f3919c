"""The boundary's stream contract, through the C ABI.

A context may be created over a caller's hipStream_t
(osm_context_create_on_stream): every operator is then ordered on that
stream, and the caller's own wait on it (hipStreamSynchronize) is the only
synchronisation needed. Copies between pinned host memory and the device can
be enqueued without waiting (osm_memcpy_*_async, osm_buffer_*_async). The
reference's context owns one queue and its copies block on a fence
(include/orbi/streammoe/backend/vulkan_compute_context.hpp:19-49,
vulkan_float_buffer.hpp:23-58); these entry points add the asynchronous
form, so the check is that the enqueued chain gives the synchronous path's
bits."""

import ctypes

import numpy as np
import pytest

import oracle as O
import osm_hip

pytestmark = pytest.mark.gpu

SEED, D, I, G, E, K, T = 33, 512, 256, 64, 32, 4, 5


def hip_runtime():
    for name in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
        try:
            lib = ctypes.CDLL(name)
            break
        except OSError:
            continue
    else:
        pytest.fail("HIP runtime library not found")
    for fn in ("hipStreamCreate", "hipStreamSynchronize", "hipStreamQuery", "hipStreamDestroy"):
        getattr(lib, fn).restype = ctypes.c_int
    lib.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    for fn in ("hipStreamSynchronize", "hipStreamQuery", "hipStreamDestroy"):
        getattr(lib, fn).argtypes = [ctypes.c_void_p]
    return lib


def build(c):
    g = osm_hip.geometry(D, I, G, osm_hip.BF16)
    slab = osm_hip.ExpertSlab(c, g, 1, E)
    slab.synthesize(SEED)
    moe = osm_hip.MoeLayer(c, g, E, K, O.synth_router_bf16(SEED, 0, E, D), osm_hip.BF16,
                           O.synth_shared_gate_bf16(SEED, 0, D), O.synth_norm_weight(SEED, 0, D),
                           O.synth_expert_blob(SEED, 0, O.SHARED_EXPERT_ID, D, I, G), max_tokens=T)
    return slab, moe


def test_context_on_caller_stream_with_async_copies(ctx):
    hip = hip_runtime()
    s = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(s)) == 0
    x = O.synth_tokens(SEED, 40, T, D).reshape(-1)
    try:
        print("[boundary] context on a caller's stream", flush=True)
        c2 = osm_hip.Context(0, stream=s.value)
        assert c2.stream == s.value
        slab, moe = build(c2)
        x_pin, y_pin = c2.pinned(np.float32, T * D), c2.pinned(np.float32, T * D)
        x_pin.array[:] = x
        xd, yd = c2.alloc(T * D * 4), c2.alloc(T * D * 4)
        for sublayer in (False, True):
            y_pin.array[:] = np.nan
            xd.upload_async(x_pin)
            moe.decode_device(slab, 0, xd.ptr, yd.ptr, T, sublayer=sublayer)
            yd.download_async(y_pin)
            assert hip.hipStreamSynchronize(s) == 0  # the caller's own wait, nothing of the library's
            got = y_pin.array.copy()

            # The same layer on the session's own-stream context, synchronous copies.
            slab1, moe1 = build(ctx)
            x1, y1 = ctx.alloc(T * D * 4), ctx.alloc(T * D * 4)
            x1.upload(x)
            moe1.decode_device(slab1, 0, x1.ptr, y1.ptr, T, sublayer=sublayer)
            ref = y1.download(np.float32, T * D)
            assert np.all(np.isfinite(ref))
            assert np.array_equal(got, ref), sublayer
            assert np.array_equal(moe.routing(T)["ids"], moe1.routing(T)["ids"])

        # Float buffer: enqueued upload and download round trip.
        fb = osm_hip.FloatBuffer(c2, T * D)
        back = c2.pinned(np.float32, T * D)
        fb.upload_async(x_pin)
        fb.download_async(back)
        assert hip.hipStreamSynchronize(s) == 0
        assert np.array_equal(back.array, x)
        lib = osm_hip.load()
        assert lib.osm_buffer_download_async(fb.h, back.ptr, T * D - 1) == osm_hip.OSM_E_INVALID
        c2.close()
        # Destroying the context leaves the caller's stream alive.
        assert hip.hipStreamQuery(s) == 0
    finally:
        assert hip.hipStreamDestroy(s) == 0


def test_context_on_stream_rejects_bad_arguments(ctx):
    lib = osm_hip.load()
    h = ctypes.c_void_p()
    assert lib.osm_context_create_on_stream(0, None, ctypes.byref(h)) == osm_hip.OSM_E_INVALID
    assert "stream is null" in osm_hip.last_error()
    assert lib.osm_context_create_on_stream(osm_hip.device_count(), ctypes.c_void_p(ctx.stream),
                                            ctypes.byref(h)) == osm_hip.OSM_E_DEVICE
    assert not h.value
