"""ctypes binding of libosm_hip.so (the C ABI declared in include/osm_hip.h).

The names mirror the reference's operator surface (run_vulkan_q4_gemv ->
run_q4_gemv, VulkanResidentExpertCache -> ExpertCache, ...) so that tests and
benchmarks read like the reference's own. Every failed call raises OsmError
carrying the library's diagnostic, the counterpart of the reference's
``executed == false`` plus ``diagnostic``.

There is no fallback: if libosm_hip.so is missing this module raises, and
every compute call runs on the HIP device.
"""

from __future__ import annotations

import ctypes
import os
import weakref
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_size_t, c_uint16, c_uint32, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libosm_hip.so")

OSM_OK, OSM_E_INVALID, OSM_E_RUNTIME, OSM_E_DEVICE = 0, 1, 2, 3
PATH_AUTO, PATH_PER_TOKEN, PATH_GROUPED = 0, 1, 2
F32, F16, BF16 = 0, 1, 2
AFFINE_Q8 = 3  # router / shared-gate dtype: MLX affine 8-bit (osm_affine_q8_c)


class OsmError(RuntimeError):
    def __init__(self, status: int, diagnostic: str):
        super().__init__(f"osm status {status}: {diagnostic}")
        self.status = status
        self.diagnostic = diagnostic


class Geometry(ctypes.Structure):
    _fields_ = [("hidden", c_uint32), ("inter", c_uint32), ("group", c_uint32), ("meta_dtype", c_uint32)]


class MoeConfig(ctypes.Structure):
    _fields_ = [
        ("geometry", Geometry),
        ("expert_count", c_uint32),
        ("top_k", c_uint32),
        ("norm_topk_prob", c_uint32),
        ("has_shared", c_uint32),
        ("rms_eps", c_float),
    ]


class MoeOutputs(ctypes.Structure):
    _fields_ = [
        ("out", c_void_p),
        ("normalized", c_void_p),
        ("ids", c_void_p),
        ("weights", c_void_p),
        ("mass", c_void_p),
        ("shared_gate", c_void_p),
        ("logits", c_void_p),
    ]


class HostCacheStats(ctypes.Structure):
    _fields_ = [(n, c_uint64) for n in ("hits", "misses", "allocated_slots", "capacity_slots", "logical_bytes", "budget_bytes")]


class ExpertCacheStats(ctypes.Structure):
    _fields_ = [(n, c_uint64) for n in ("hits", "misses", "loads", "evictions", "resident_entries", "resident_bytes", "budget_bytes")]


READ_EXPERTS_FN = ctypes.CFUNCTYPE(c_int, c_void_p, POINTER(c_uint32), POINTER(c_uint32), POINTER(c_void_p), c_size_t, c_size_t)

_H = c_void_p  # opaque handle
_PROTOTYPES = {
    "osm_last_error": (c_char_p, []),
    "osm_device_count": (c_int, [POINTER(c_int)]),
    "osm_context_create": (c_int, [c_int, POINTER(_H)]),
    "osm_context_create_on_stream": (c_int, [c_int, c_void_p, POINTER(_H)]),
    "osm_context_destroy": (None, [_H]),
    "osm_context_synchronize": (c_int, [_H]),
    "osm_context_device_name": (c_int, [_H, c_char_p, c_size_t]),
    "osm_context_stream": (c_void_p, [_H]),
    "osm_event_create": (c_int, [_H, POINTER(_H)]),
    "osm_event_destroy": (None, [_H]),
    "osm_event_record": (c_int, [_H]),
    "osm_event_elapsed_ms": (c_int, [_H, _H, POINTER(c_float)]),
    "osm_device_alloc": (c_int, [_H, c_size_t, POINTER(c_void_p)]),
    "osm_device_free": (c_int, [_H, c_void_p]),
    "osm_memcpy_h2d": (c_int, [_H, c_void_p, c_void_p, c_size_t]),
    "osm_memcpy_d2h": (c_int, [_H, c_void_p, c_void_p, c_size_t]),
    "osm_memcpy_h2d_async": (c_int, [_H, c_void_p, c_void_p, c_size_t]),
    "osm_memcpy_d2h_async": (c_int, [_H, c_void_p, c_void_p, c_size_t]),
    "osm_host_alloc": (c_int, [_H, c_size_t, POINTER(c_void_p)]),
    "osm_host_free": (c_int, [_H, c_void_p]),
    "osm_buffer_create": (c_int, [_H, c_size_t, POINTER(_H)]),
    "osm_buffer_destroy": (None, [_H]),
    "osm_buffer_size": (c_size_t, [_H]),
    "osm_buffer_device_ptr": (c_void_p, [_H]),
    "osm_buffer_upload": (c_int, [_H, c_void_p, c_size_t]),
    "osm_buffer_download": (c_int, [_H, c_void_p, c_size_t]),
    "osm_buffer_upload_async": (c_int, [_H, c_void_p, c_size_t]),
    "osm_buffer_download_async": (c_int, [_H, c_void_p, c_size_t]),
    "osm_q4_dequant": (c_int, [_H, c_void_p, c_size_t, c_size_t, c_size_t, c_void_p, c_void_p, c_size_t, c_size_t, c_void_p, c_size_t]),
    "osm_q4_gemv": (c_int, [_H, c_void_p, c_size_t, c_size_t, c_size_t, c_void_p, c_void_p, c_size_t, c_size_t, c_void_p, c_size_t, c_void_p, c_size_t]),
    "osm_swiglu": (c_int, [_H, c_void_p, c_size_t, c_void_p, c_size_t, c_void_p]),
    "osm_rms_norm": (c_int, [_H, c_void_p, c_size_t, c_size_t, c_size_t, c_void_p, c_size_t, c_float, c_void_p]),
    "osm_unpack_nibbles": (c_int, [_H, c_void_p, c_size_t, c_void_p]),
    "osm_q4_quantize": (c_int, [_H, c_void_p, c_size_t, c_size_t, c_size_t, c_void_p, c_void_p, c_void_p, POINTER(c_float), POINTER(ctypes.c_double)]),
    "osm_q4_gemv_buffers": (c_int, [_H, c_void_p, c_size_t, c_size_t, c_size_t, c_void_p, c_void_p, c_size_t, c_size_t, _H, _H]),
    "osm_q4_projection_create": (c_int, [_H, c_void_p, c_size_t, c_size_t, c_size_t, c_void_p, c_void_p, c_uint32, c_size_t, POINTER(_H)]),
    "osm_q4_projection_destroy": (None, [_H]),
    "osm_q4_gemv_preloaded": (c_int, [_H, _H, _H, _H]),
    "osm_swiglu_buffers": (c_int, [_H, _H, _H, _H]),
    "osm_weighted_accumulate": (c_int, [_H, _H, c_float, _H]),
    "osm_expert_blob_bytes": (c_size_t, [POINTER(Geometry)]),
    "osm_expert_create": (c_int, [_H, c_void_p, c_size_t, POINTER(Geometry), POINTER(_H)]),
    "osm_expert_destroy": (None, [_H]),
    "osm_expert_run": (c_int, [_H, _H, c_void_p, c_size_t, c_void_p, c_size_t]),
    "osm_expert_run_from_buffer": (c_int, [_H, _H, _H]),
    "osm_expert_download_output": (c_int, [_H, c_void_p, c_size_t]),
    "osm_expert_accounted_bytes": (c_size_t, [_H]),
    "osm_shared_expert_create": (c_int, [_H, c_void_p, c_size_t, POINTER(Geometry), c_void_p, c_size_t, POINTER(_H)]),
    "osm_shared_expert_destroy": (None, [_H]),
    "osm_shared_expert_scalar_scale": (c_int, [_H, c_void_p, c_size_t, POINTER(c_float)]),
    "osm_shared_expert_run_from_buffer": (c_int, [_H, _H, _H]),
    "osm_shared_expert_download_output": (c_int, [_H, c_void_p, c_size_t]),
    "osm_expert_slab_create": (c_int, [_H, POINTER(Geometry), c_uint32, c_uint32, POINTER(_H)]),
    "osm_expert_slab_destroy": (None, [_H]),
    "osm_expert_slab_stride": (c_size_t, [_H]),
    "osm_expert_slab_upload": (c_int, [_H, c_uint32, c_uint32, c_void_p, c_size_t]),
    "osm_expert_slab_download": (c_int, [_H, c_uint32, c_uint32, c_void_p, c_size_t]),
    "osm_expert_slab_synthesize": (c_int, [_H, c_uint64]),
    "osm_moe_layer_create": (c_int, [_H, POINTER(MoeConfig), c_void_p, c_uint32, c_void_p, c_void_p, c_void_p, c_size_t, c_uint32, POINTER(_H)]),
    "osm_moe_layer_destroy": (None, [_H]),
    "osm_moe_layer_run_slab": (c_int, [_H, _H, _H, c_uint32, c_void_p, c_uint32, c_int, POINTER(MoeOutputs)]),
    "osm_moe_layer_run_cached": (c_int, [_H, _H, _H, c_uint32, c_void_p, c_uint32, c_int, POINTER(MoeOutputs)]),
    "osm_moe_layer_run_cached_picks": (c_int, [_H, _H, _H, c_uint32, c_void_p, c_uint32, c_int, c_void_p, c_void_p, POINTER(MoeOutputs)]),
    "osm_moe_layer_decode_device": (c_int, [_H, _H, _H, c_uint32, c_void_p, c_void_p, c_uint32, c_int]),
    "osm_moe_layer_decode_device_static": (c_int, [_H, _H, _H, c_uint32, c_void_p, c_void_p, c_uint32, c_int]),
    "osm_moe_layer_static_tokens_capacity": (c_uint32, [_H]),
    "osm_moe_decode_layers": (c_int, [_H, POINTER(_H), POINTER(c_uint32), c_uint32, _H, c_void_p, c_void_p, c_void_p, c_uint32, c_int]),
    "osm_moe_layer_launch_phase": (c_int, [_H, _H, _H, c_uint32, c_void_p, c_void_p, c_uint32, c_int, c_int]),
    "osm_moe_layer_set_path": (c_int, [_H, c_int]),
    "osm_moe_layer_prefill_device": (c_int, [_H, _H, _H, c_uint32, c_void_p, c_void_p, c_uint32]),
    "osm_moe_layer_routing": (c_int, [_H, _H, c_uint32, POINTER(MoeOutputs)]),
    "osm_moe_layer_routing_stats": (c_int, [_H, _H, POINTER(c_uint32), c_int]),
    "osm_libm_expf_checksums": (c_int, [_H, c_uint32, c_uint64, c_uint32, c_void_p]),
    "osm_decode_graph_create": (c_int, [_H, POINTER(_H), POINTER(c_uint32), c_uint32, _H, c_void_p, c_void_p, c_void_p, c_uint32, c_int, POINTER(_H)]),
    "osm_graph_capture_begin": (c_int, [_H]),
    "osm_graph_capture_end": (c_int, [_H, POINTER(_H)]),
    "osm_graph_launch": (c_int, [_H, _H]),
    "osm_graph_destroy": (None, [_H]),
    "osm_memcpy_d2d_async": (c_int, [_H, c_void_p, c_void_p, c_size_t]),
    "osm_expert_store_create": (c_int, [POINTER(Geometry), c_uint32, c_uint32, POINTER(_H)]),
    "osm_expert_store_destroy": (None, [_H]),
    "osm_expert_store_blob": (c_void_p, [_H, c_uint32, c_uint32]),
    "osm_expert_store_synthesize": (c_int, [_H, _H, c_uint64]),
    "osm_host_cache_create": (c_int, [c_size_t, c_size_t, c_size_t, c_int, READ_EXPERTS_FN, c_void_p, POINTER(_H)]),
    "osm_host_cache_destroy": (None, [_H]),
    "osm_host_cache_create_with_storage": (c_int, [_H, c_size_t, c_size_t, c_int, POINTER(_H)]),
    "osm_pread_storage_create": (c_int, [c_char_p, c_uint32, c_uint32, c_size_t, POINTER(_H)]),
    "osm_moe_run_cached_layers": (c_int, [_H, c_void_p, c_void_p, c_uint32, _H, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p]),
    "osm_qpack_expert_repack": (c_int, [POINTER(Geometry), c_void_p, c_size_t, c_uint64, c_void_p, c_void_p, c_size_t, POINTER(c_int)]),
    "osm_qpack_open": (c_int, [c_char_p, POINTER(_H)]),
    "osm_qpack_close": (None, [_H]),
    "osm_qpack_get_info": (c_int, [_H, c_void_p]),
    "osm_qpack_get_section": (c_int, [_H, c_uint32, c_void_p]),
    "osm_qpack_find_section": (c_int, [_H, c_char_p, c_void_p]),
    "osm_qpack_section_shape": (c_int, [_H, c_uint32, c_void_p, c_uint32, POINTER(c_uint32)]),
    "osm_qpack_linear_layers": (c_int, [_H, c_void_p, c_size_t]),
    "osm_qpack_file_size": (c_int, [_H, c_char_p, POINTER(c_uint64)]),
    "osm_qpack_read_expert": (c_int, [_H, c_uint32, c_uint32, c_void_p, c_size_t]),
    "osm_qpack_storage_create": (c_int, [c_char_p, c_void_p, POINTER(_H)]),
    "osm_expert_storage_destroy": (None, [_H]),
    "osm_expert_storage_stride": (c_size_t, [_H]),
    "osm_expert_storage_read": (c_int, [_H, c_void_p, c_void_p, c_void_p, c_size_t, c_size_t]),
    "osm_host_cache_fetch": (c_int, [_H, c_uint32, c_void_p, c_size_t, c_void_p, c_void_p]),
    "osm_host_cache_resident_slot": (c_int64, [_H, c_uint32, c_uint32]),
    "osm_host_cache_stats_get": (None, [_H, POINTER(HostCacheStats)]),
    "osm_expert_cache_create_from_store": (c_int, [_H, _H, c_size_t, POINTER(_H)]),
    "osm_expert_cache_create_from_host_cache": (c_int, [_H, _H, POINTER(Geometry), c_size_t, POINTER(_H)]),
    "osm_expert_cache_destroy": (None, [_H]),
    "osm_expert_cache_get": (c_int, [_H, c_uint32, c_uint32, POINTER(c_void_p)]),
    "osm_expert_cache_run": (c_int, [_H, c_uint32, c_uint32, c_void_p, c_size_t, c_void_p, c_size_t]),
    "osm_expert_cache_contains": (c_int, [_H, c_uint32, c_uint32]),
    "osm_expert_cache_stats_get": (None, [_H, POINTER(ExpertCacheStats)]),
    "osm_expert_cache_bytes_filled": (c_uint64, [_H]),
    "osm_cache_policy_create": (c_int, [c_size_t, POINTER(_H)]),
    "osm_cache_policy_destroy": (None, [_H]),
    "osm_cache_policy_get": (c_int, [_H, c_uint32, c_uint32, c_size_t, c_void_p, c_size_t, POINTER(c_size_t)]),
    "osm_cache_policy_contains": (c_int, [_H, c_uint32, c_uint32]),
    "osm_cache_policy_stats_get": (None, [_H, POINTER(ExpertCacheStats)]),
    "osm_synth_expert_blob": (c_int, [_H, c_uint64, c_uint32, c_uint32, POINTER(Geometry), c_void_p, c_size_t]),
    "osm_synth_router_bf16": (c_int, [_H, c_uint64, c_uint32, c_uint32, c_uint32, c_void_p]),
    "osm_synth_shared_gate_bf16": (c_int, [_H, c_uint64, c_uint32, c_uint32, c_void_p]),
    "osm_synth_norm_weight": (c_int, [_H, c_uint64, c_uint32, c_uint32, c_void_p]),
    "osm_synth_tokens": (c_int, [_H, c_uint64, c_uint32, c_uint32, c_uint32, c_void_p]),
    "osm_synth_tokens_device": (c_int, [_H, c_uint64, c_uint32, c_uint32, c_uint32, c_void_p]),
}

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads libosm_hip.so once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise OsmError(OSM_E_RUNTIME, f"{path} is not built (run __graft_entry__.build() or make -C orbi-streammoe_amd)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols() -> list:
    return list(_PROTOTYPES)


def last_error() -> str:
    return load().osm_last_error().decode(errors="replace")


def check(status: int) -> None:
    if status != OSM_OK:
        raise OsmError(status, last_error())


def _p(a: np.ndarray) -> c_void_p:
    return c_void_p(a.ctypes.data)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def device_count() -> int:
    n = c_int(0)
    st = load().osm_device_count(ctypes.byref(n))
    return n.value if st == OSM_OK else 0


def libm_expf_checksums(ctx, first_bits: int, count: int, block: int) -> np.ndarray:
    """Block checksums of the selection's exp on the device over float bit
    patterns first_bits .. first_bits + count - 1 (osm_libm_expf_checksums)."""
    out = np.zeros((count + block - 1) // block, np.uint64)
    check(load().osm_libm_expf_checksums(ctx.h, first_bits, count, block, _p(out)))
    return out


def geometry(hidden: int, inter: int, group: int = 64, meta_dtype: int = BF16) -> Geometry:
    return Geometry(hidden, inter, group, meta_dtype)


def expert_blob_bytes(g: Geometry) -> int:
    return load().osm_expert_blob_bytes(ctypes.byref(g))


class _Handle:
    _destroy = None

    def __init__(self, h):
        self.h = h

    def close(self):
        if self.h is not None and self.h.value:
            getattr(load(), self._destroy)(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


# ---- context / events / memory ------------------------------------------------------
class Context(_Handle):
    """HipComputeContext: one device, a compute stream and a fill stream.

    The library's objects must not outlive the context they were created on
    (the resident cache, for one, keeps using its streams until it is
    destroyed). close() therefore closes every handle still open on this
    context first, newest first, then the context."""

    _destroy = "osm_context_destroy"

    def __init__(self, device: int = 0, stream=None):
        """stream: None for a stream of the context's own, else a caller's
        hipStream_t (an int or c_void_p) on `device` that every operator of
        the context is then ordered on; the caller keeps it alive."""
        self._children = []
        h = c_void_p()
        if stream is None:
            check(load().osm_context_create(device, ctypes.byref(h)))
        else:
            check(load().osm_context_create_on_stream(device, c_void_p(int(stream) if not isinstance(stream, c_void_p) else stream.value), ctypes.byref(h)))
        super().__init__(h)

    def _adopt(self, child):
        self._children = [r for r in self._children if r() is not None]
        self._children.append(weakref.ref(child))

    def close(self):
        for ref in reversed(getattr(self, "_children", [])):
            child = ref()
            if child is not None:
                child.close()
        self._children = []
        super().close()

    def synchronize(self):
        check(load().osm_context_synchronize(self.h))

    @property
    def device_name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        check(load().osm_context_device_name(self.h, buf, 256))
        return buf.value.decode()

    def alloc(self, nbytes: int) -> "DeviceArray":
        return DeviceArray(self, nbytes)

    def pinned(self, dtype, count) -> "PinnedArray":
        return PinnedArray(self, dtype, count)

    @property
    def stream(self) -> int:
        """The hipStream_t every operator of this context is ordered on."""
        return load().osm_context_stream(self.h) or 0

    def copy_d2d(self, dst_ptr, src_ptr, nbytes: int):
        """Enqueued device-to-device copy on the compute stream (no sync)."""
        check(load().osm_memcpy_d2d_async(self.h, dst_ptr, src_ptr, nbytes))

    def capture(self) -> "_Capture":
        return _Capture(self)

    def event(self) -> "Event":
        return Event(self)


class Event(_Handle):
    _destroy = "osm_event_destroy"

    def __init__(self, ctx: Context):
        h = c_void_p()
        check(load().osm_event_create(ctx.h, ctypes.byref(h)))
        super().__init__(h)
        ctx._adopt(self)

    def record(self):
        check(load().osm_event_record(self.h))

    def elapsed_ms(self, stop: "Event") -> float:
        ms = c_float(0)
        check(load().osm_event_elapsed_ms(self.h, stop.h, ctypes.byref(ms)))
        return ms.value


class DeviceArray:
    """Raw device allocation (for device-pointer entry points)."""

    def __init__(self, ctx: Context, nbytes: int):
        self.ctx = ctx
        self.nbytes = nbytes
        p = c_void_p()
        check(load().osm_device_alloc(ctx.h, nbytes, ctypes.byref(p)))
        self.ptr = p
        ctx._adopt(self)

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(load().osm_memcpy_h2d(self.ctx.h, self.ptr, _p(a), a.nbytes))

    def download(self, dtype, count) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(load().osm_memcpy_d2h(self.ctx.h, _p(out), self.ptr, out.nbytes))
        return out

    def upload_async(self, src: "PinnedArray", count=None):
        """Enqueued copy from pinned host memory; src must stay unchanged
        until the context's stream has passed it."""
        n = src.array.nbytes if count is None else count * src.array.itemsize
        assert n <= self.nbytes
        check(load().osm_memcpy_h2d_async(self.ctx.h, self.ptr, src.ptr, n))

    def download_async(self, dst: "PinnedArray", count=None):
        """Enqueued copy into pinned host memory, valid after the context's
        stream has passed it."""
        n = dst.array.nbytes if count is None else count * dst.array.itemsize
        assert n <= self.nbytes
        check(load().osm_memcpy_d2h_async(self.ctx.h, dst.ptr, self.ptr, n))

    def close(self):
        if self.ptr is not None and self.ptr.value:
            check(load().osm_device_free(self.ctx.h, self.ptr))
        self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class PinnedArray:
    """Page-locked host memory (osm_host_alloc) seen as a numpy array: the
    source or target of asynchronous copies."""

    def __init__(self, ctx: Context, dtype, count: int):
        self.ctx = ctx
        dt = np.dtype(dtype)
        p = c_void_p()
        check(load().osm_host_alloc(ctx.h, max(1, count * dt.itemsize), ctypes.byref(p)))
        self.ptr = p
        buf = (ctypes.c_char * (count * dt.itemsize)).from_address(p.value)
        self.array = np.frombuffer(buf, dtype=dt, count=count)
        ctx._adopt(self)

    def close(self):
        if self.ptr is not None and self.ptr.value:
            self.array = None
            check(load().osm_host_free(self.ctx.h, self.ptr))
        self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class FloatBuffer(_Handle):
    """VulkanFloatBuffer counterpart."""

    _destroy = "osm_buffer_destroy"

    def __init__(self, ctx: Context, count: int):
        h = c_void_p()
        check(load().osm_buffer_create(ctx.h, count, ctypes.byref(h)))
        super().__init__(h)
        ctx._adopt(self)
        self.count = count

    def upload(self, values):
        v = _c(values, np.float32)
        check(load().osm_buffer_upload(self.h, _p(v), v.size))

    def download(self) -> np.ndarray:
        out = np.empty(self.count, np.float32)
        check(load().osm_buffer_download(self.h, _p(out), out.size))
        return out

    def upload_async(self, src: PinnedArray):
        check(load().osm_buffer_upload_async(self.h, src.ptr, src.array.size))

    def download_async(self, dst: PinnedArray):
        check(load().osm_buffer_download_async(self.h, dst.ptr, dst.array.size))


# ---- single operators ----------------------------------------------------------------
def run_q4_dequant(ctx, packed, rows, packed_cols, scales, biases, group_size) -> np.ndarray:
    pk, s, b = _c(packed, np.uint32), _c(scales, np.float32), _c(biases, np.float32)
    out = np.empty(rows * packed_cols * 8, np.float32)
    check(load().osm_q4_dequant(ctx.h, _p(pk), pk.size, rows, packed_cols, _p(s), _p(b), s.size, group_size, _p(out), out.size))
    return out


def run_q4_gemv(ctx, packed, out_dim, packed_cols, scales, biases, group_size, x) -> np.ndarray:
    pk, s, b, xv = _c(packed, np.uint32), _c(scales, np.float32), _c(biases, np.float32), _c(x, np.float32)
    y = np.empty(out_dim, np.float32)
    if s.size != b.size:
        raise OsmError(OSM_E_INVALID, "scale/bias size mismatch")
    check(load().osm_q4_gemv(ctx.h, _p(pk), pk.size, out_dim, packed_cols, _p(s), _p(b), s.size, group_size, _p(xv), xv.size, _p(y), y.size))
    return y


def run_q4_gemv_buffers(ctx, packed, out_dim, packed_cols, scales, biases, group_size, x: FloatBuffer, y: FloatBuffer):
    pk, s, b = _c(packed, np.uint32), _c(scales, np.float32), _c(biases, np.float32)
    check(load().osm_q4_gemv_buffers(ctx.h, _p(pk), pk.size, out_dim, packed_cols, _p(s), _p(b), s.size, group_size, x.h, y.h))


def run_swiglu(ctx, gate, up) -> np.ndarray:
    g, u = _c(gate, np.float32), _c(up, np.float32)
    out = np.empty(g.size, np.float32)
    check(load().osm_swiglu(ctx.h, _p(g), g.size, _p(u), u.size, _p(out)))
    return out


def run_rms_norm(ctx, values, rows, dim, weight, eps) -> np.ndarray:
    v, w = _c(values, np.float32), _c(weight, np.float32)
    out = np.empty(v.size, np.float32)
    check(load().osm_rms_norm(ctx.h, _p(v), v.size, rows, dim, _p(w), w.size, eps, _p(out)))
    return out


def unpack_nibbles(ctx, packed) -> np.ndarray:
    pk = _c(packed, np.uint32)
    out = np.empty(pk.size * 8, np.uint8)
    check(load().osm_unpack_nibbles(ctx.h, _p(pk), pk.size, _p(out)))
    return out


def q4_quantize(ctx, values, group):
    """quantize_affine_q4_rows on the device: (packed, scales, biases, max_err, mean_err)."""
    v = _c(values, np.float32)
    if v.ndim != 2:
        raise ValueError("values must be [rows, cols]")
    rows, cols = v.shape
    packed = np.empty(max(rows * (cols // 8), 1), np.uint32)
    ng = rows * (cols // group) if group and cols % group == 0 else 1
    scales = np.empty(max(ng, 1), np.float32)
    biases = np.empty_like(scales)
    mx, mean = c_float(0), ctypes.c_double(0)
    check(load().osm_q4_quantize(ctx.h, _p(v), rows, cols, group, _p(packed), _p(scales), _p(biases),
                                 ctypes.byref(mx), ctypes.byref(mean)))
    return packed, scales, biases, mx.value, mean.value


class Q4ProjectionWeights(_Handle):
    _destroy = "osm_q4_projection_destroy"

    def __init__(self, ctx, packed, out_dim, packed_cols, scales, biases, group_size, meta_dtype=F32):
        pk = _c(packed, np.uint32)
        dt = {F32: np.float32, F16: np.float16, BF16: np.uint16}[meta_dtype]
        s, b = _c(scales, dt), _c(biases, dt)
        h = c_void_p()
        check(load().osm_q4_projection_create(ctx.h, _p(pk), pk.size, out_dim, packed_cols, _p(s), _p(b), meta_dtype, group_size, ctypes.byref(h)))
        super().__init__(h)
        ctx._adopt(self)


def run_q4_gemv_preloaded(ctx, weights: Q4ProjectionWeights, x: FloatBuffer, y: FloatBuffer):
    check(load().osm_q4_gemv_preloaded(ctx.h, weights.h, x.h, y.h))


def run_swiglu_buffers(ctx, gate: FloatBuffer, up: FloatBuffer, out: FloatBuffer):
    check(load().osm_swiglu_buffers(ctx.h, gate.h, up.h, out.h))


def run_weighted_accumulate(ctx, source: FloatBuffer, weight: float, accumulator: FloatBuffer):
    check(load().osm_weighted_accumulate(ctx.h, source.h, float(weight), accumulator.h))


# ---- experts ---------------------------------------------------------------------------
class ResidentExpert(_Handle):
    """VulkanResidentExpert counterpart over one expert blob."""

    _destroy = "osm_expert_destroy"

    def __init__(self, ctx, blob: np.ndarray, g: Geometry):
        bl = np.ascontiguousarray(blob).view(np.uint8)
        h = c_void_p()
        check(load().osm_expert_create(ctx.h, _p(bl), bl.size, ctypes.byref(g), ctypes.byref(h)))
        super().__init__(h)
        ctx._adopt(self)
        self.ctx, self.g = ctx, g

    def run(self, x) -> np.ndarray:
        xv = _c(x, np.float32)
        out = np.empty(self.g.hidden, np.float32)
        check(load().osm_expert_run(self.ctx.h, self.h, _p(xv), xv.size, _p(out), out.size))
        return out

    def run_from_buffer(self, x: FloatBuffer):
        check(load().osm_expert_run_from_buffer(self.ctx.h, self.h, x.h))

    def output(self) -> np.ndarray:
        out = np.empty(self.g.hidden, np.float32)
        check(load().osm_expert_download_output(self.h, _p(out), out.size))
        return out

    @property
    def accounted_bytes(self) -> int:
        return load().osm_expert_accounted_bytes(self.h)


class SharedExpert(_Handle):
    _destroy = "osm_shared_expert_destroy"

    def __init__(self, ctx, blob, g: Geometry, scalar_gate):
        bl = np.ascontiguousarray(blob).view(np.uint8)
        sg = _c(scalar_gate, np.float32)
        h = c_void_p()
        check(load().osm_shared_expert_create(ctx.h, _p(bl), bl.size, ctypes.byref(g), _p(sg), sg.size, ctypes.byref(h)))
        super().__init__(h)
        ctx._adopt(self)
        self.ctx, self.g = ctx, g

    def scalar_scale(self, hidden) -> float:
        xv = _c(hidden, np.float32)
        out = c_float(0)
        check(load().osm_shared_expert_scalar_scale(self.h, _p(xv), xv.size, ctypes.byref(out)))
        return out.value

    def run_from_buffer(self, hidden: FloatBuffer):
        check(load().osm_shared_expert_run_from_buffer(self.ctx.h, self.h, hidden.h))

    def output(self) -> np.ndarray:
        out = np.empty(self.g.hidden, np.float32)
        check(load().osm_shared_expert_download_output(self.h, _p(out), out.size))
        return out


class ExpertSlab(_Handle):
    """All experts of `layers` layers resident in one HBM slab."""

    _destroy = "osm_expert_slab_destroy"

    def __init__(self, ctx, g: Geometry, layers: int, experts: int):
        h = c_void_p()
        check(load().osm_expert_slab_create(ctx.h, ctypes.byref(g), layers, experts, ctypes.byref(h)))
        super().__init__(h)
        ctx._adopt(self)
        self.ctx, self.g, self.layers, self.experts = ctx, g, layers, experts
        self.stride = load().osm_expert_slab_stride(h)

    def upload(self, layer, expert, blob):
        bl = np.ascontiguousarray(blob).view(np.uint8)
        check(load().osm_expert_slab_upload(self.h, layer, expert, _p(bl), bl.size))

    def download(self, layer, expert) -> np.ndarray:
        out = np.empty(self.stride, np.uint8)
        check(load().osm_expert_slab_download(self.h, layer, expert, _p(out), out.size))
        return out

    def synthesize(self, seed: int):
        check(load().osm_expert_slab_synthesize(self.h, seed))


class AffineQ8(ctypes.Structure):
    """osm_affine_q8_c: one MLX affine 8-bit matrix [rows, cols]."""

    _fields_ = [("packed", c_void_p), ("scales", c_void_p), ("biases", c_void_p), ("group", c_uint32)]

    @classmethod
    def of(cls, packed, scales, biases, group):
        arrs = (_c(packed, np.uint32), _c(scales, np.float32), _c(biases, np.float32))
        obj = cls(arrs[0].ctypes.data, arrs[1].ctypes.data, arrs[2].ctypes.data, group)
        obj._arrays = arrs  # the views must outlive the struct
        return obj


class MoeLayer(_Handle):
    """Layer state of QwenCheckpointSparseMoeLayer / QwenCheckpointMoeSublayer.
    router_dtype AFFINE_Q8: router and shared_gate_vec are (packed, scales,
    biases, group) tuples of [E, D] and [1, D] 8-bit matrices."""

    _destroy = "osm_moe_layer_destroy"

    def __init__(self, ctx, g: Geometry, expert_count, top_k, router, router_dtype=BF16, shared_gate_vec=None,
                 norm_weight=None, shared_blob=None, max_tokens=1, norm_topk_prob=True, rms_eps=1e-6):
        has_shared = shared_blob is not None
        cfg = MoeConfig(g, expert_count, top_k, 1 if norm_topk_prob else 0, 1 if has_shared else 0, rms_eps)
        if router_dtype == AFFINE_Q8:
            r = AffineQ8.of(*router)
            sg = AffineQ8.of(*shared_gate_vec) if shared_gate_vec is not None else None
            rp = ctypes.cast(ctypes.pointer(r), c_void_p)
            sp = ctypes.cast(ctypes.pointer(sg), c_void_p) if sg is not None else None
        else:
            rdt = {F32: np.float32, F16: np.float16, BF16: np.uint16}[router_dtype]
            r = _c(router, rdt)
            sg = _c(shared_gate_vec, rdt) if shared_gate_vec is not None else None
            rp, sp = _p(r), (_p(sg) if sg is not None else None)
        nw = _c(norm_weight, np.float32) if norm_weight is not None else None
        sb = np.ascontiguousarray(shared_blob).view(np.uint8) if has_shared else None
        h = c_void_p()
        check(load().osm_moe_layer_create(
            ctx.h, ctypes.byref(cfg), rp, router_dtype, sp,
            _p(nw) if nw is not None else None, _p(sb) if sb is not None else None,
            sb.size if sb is not None else 0, max_tokens, ctypes.byref(h)))
        super().__init__(h)
        ctx._adopt(self)
        self.ctx, self.g, self.E, self.k, self.max_tokens = ctx, g, expert_count, top_k, max_tokens
        self._keep = (r, sg, nw, sb)

    def _outputs(self, tokens, sublayer):
        D, E, K = self.g.hidden, self.E, self.k
        res = {
            "out": np.empty((tokens, D), np.float32),
            "normalized": np.empty((tokens, D), np.float32) if sublayer else None,
            "ids": np.empty((tokens, K), np.uint32),
            "weights": np.empty((tokens, K), np.float32),
            "mass": np.empty(tokens, np.float32),
            "shared_gate": np.empty(tokens, np.float32),
            "logits": np.empty((tokens, E), np.float32),
        }
        o = MoeOutputs(*[(_p(v) if v is not None else None) for v in (res["out"], res["normalized"], res["ids"], res["weights"], res["mass"], res["shared_gate"], res["logits"])])
        return res, o

    def run_slab(self, slab: ExpertSlab, slab_layer, hidden, sublayer=False) -> dict:
        x = _c(hidden, np.float32).reshape(-1, self.g.hidden)
        res, o = self._outputs(x.shape[0], sublayer)
        check(load().osm_moe_layer_run_slab(self.ctx.h, self.h, slab.h, slab_layer, _p(x), x.shape[0], 1 if sublayer else 0, ctypes.byref(o)))
        return res

    def run_cached(self, cache: "ExpertCache", layer, hidden, sublayer=False, picks=None) -> dict:
        """picks: None (route), or (ids [tokens, k] uint32, weights [tokens, k] float32)."""
        x = _c(hidden, np.float32).reshape(-1, self.g.hidden)
        res, o = self._outputs(x.shape[0], sublayer)
        if picks is None:
            check(load().osm_moe_layer_run_cached(self.ctx.h, self.h, cache.h, layer, _p(x), x.shape[0], 1 if sublayer else 0, ctypes.byref(o)))
        else:
            ids = _c(picks[0], np.uint32)
            w = _c(picks[1], np.float32)
            check(load().osm_moe_layer_run_cached_picks(self.ctx.h, self.h, cache.h, layer, _p(x), x.shape[0], 1 if sublayer else 0,
                                                        _p(ids), _p(w), ctypes.byref(o)))
        return res

    def decode_device(self, slab, slab_layer, x_ptr, y_ptr, tokens, sublayer=False):
        check(load().osm_moe_layer_decode_device(self.ctx.h, self.h, slab.h, slab_layer, x_ptr, y_ptr, tokens, 1 if sublayer else 0))

    def decode_device_static(self, slab, slab_layer, x_ptr, y_ptr, tokens, sublayer=False):
        """decode_device with no device allocation: the per-token kernels with
        their workspace in the library's fixed per-device array."""
        check(load().osm_moe_layer_decode_device_static(self.ctx.h, self.h, slab.h, slab_layer, x_ptr, y_ptr, tokens,
                                                        1 if sublayer else 0))

    @property
    def static_tokens_capacity(self) -> int:
        return int(load().osm_moe_layer_static_tokens_capacity(self.h))

    def set_path(self, path):
        """PATH_AUTO, PATH_PER_TOKEN or PATH_GROUPED."""
        check(load().osm_moe_layer_set_path(self.h, path))

    def prefill_device(self, slab, slab_layer, x_bf16_ptr, y_ptr, tokens):
        check(load().osm_moe_layer_prefill_device(self.ctx.h, self.h, slab.h, slab_layer, x_bf16_ptr, y_ptr, tokens))

    def routing(self, tokens, normalized=False) -> dict:
        """Routing of the layer's last call (device-side decodes and prefill
        return only y): ids, weights, mass, shared gate, logits and, when
        asked, the normalised input."""
        res, o = self._outputs(tokens, normalized)
        del res["out"]
        o.out = None
        check(load().osm_moe_layer_routing(self.ctx.h, self.h, tokens, ctypes.byref(o)))
        return res

    def routing_stats(self, reset=False) -> dict:
        """Selections, those that took the exact path, exact paths over every
        expert, and the adjacent near ties (exps close enough for their
        probabilities to round to one value, the higher id first) that sent a
        selection to the recompute over every expert, since creation or a
        reset."""
        v = (c_uint32 * 4)()
        check(load().osm_moe_layer_routing_stats(self.ctx.h, self.h, v, 1 if reset else 0))
        return dict(zip(("selections", "exact", "exact_all", "near_ties"), list(v)))

    def launch_phase(self, slab, slab_layer, x_ptr, y_ptr, tokens, sublayer, phase):
        check(load().osm_moe_layer_launch_phase(self.ctx.h, self.h, slab.h, slab_layer, x_ptr, y_ptr, tokens, 1 if sublayer else 0, phase))


def decode_layers(ctx, layers, slab_layers, slab, x_ptr, y_ptr, scratch_ptr, tokens, chained):
    n = len(layers)
    arr = (c_void_p * n)(*[l.h for l in layers])
    sl = (c_uint32 * n)(*slab_layers)
    check(load().osm_moe_decode_layers(ctx.h, arr, sl, n, slab.h, x_ptr, y_ptr, scratch_ptr, tokens, 1 if chained else 0))


class Graph(_Handle):
    """Work recorded once from a context's compute stream into a HIP graph;
    launch() replays it. Whatever it reads and writes must outlive it."""

    _destroy = "osm_graph_destroy"

    def __init__(self, ctx, h, keep=()):
        super().__init__(h)
        ctx._adopt(self)
        self.ctx = ctx
        self._keep = keep

    def launch(self):
        check(load().osm_graph_launch(self.ctx.h, self.h))


def decode_graph(ctx, layers, slab_layers, slab, x_ptr, y_ptr, scratch_ptr, tokens, chained) -> Graph:
    """decode_layers(...) with these exact arguments, captured into a graph."""
    n = len(layers)
    arr = (c_void_p * n)(*[l.h for l in layers])
    sl = (c_uint32 * n)(*slab_layers)
    h = c_void_p()
    check(load().osm_decode_graph_create(ctx.h, arr, sl, n, slab.h, x_ptr, y_ptr, scratch_ptr, tokens,
                                         1 if chained else 0, ctypes.byref(h)))
    return Graph(ctx, h, (layers, slab))


class _Capture:
    """`with ctx.capture() as cap:` records the enqueue-only calls made inside
    on ctx; cap.graph is the instantiated graph afterwards."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.graph = None

    def __enter__(self):
        check(load().osm_graph_capture_begin(self.ctx.h))
        return self

    def __exit__(self, exc_type, exc, tb):
        h = c_void_p()
        rc = load().osm_graph_capture_end(self.ctx.h, ctypes.byref(h))  # always ends the capture
        if exc_type is None:
            check(rc)
            self.graph = Graph(self.ctx, h)
        elif rc == 0:
            load().osm_graph_destroy(h)
        return False


# ---- sources and caches -------------------------------------------------------------
class ExpertStore(_Handle):
    """Whole model in pinned host memory (fill source of the capped cache)."""

    _destroy = "osm_expert_store_destroy"

    def __init__(self, g: Geometry, layers, experts):
        h = c_void_p()
        check(load().osm_expert_store_create(ctypes.byref(g), layers, experts, ctypes.byref(h)))
        super().__init__(h)
        self.g, self.layers, self.experts = g, layers, experts
        self.stride = expert_blob_bytes(g)

    def blob_view(self, layer, expert) -> np.ndarray:
        p = load().osm_expert_store_blob(self.h, layer, expert)
        if not p:
            raise OsmError(OSM_E_INVALID, "expert store index out of range")
        return np.ctypeslib.as_array((ctypes.c_uint8 * self.stride).from_address(p))

    def synthesize(self, ctx, seed):
        check(load().osm_expert_store_synthesize(ctx.h, self.h, seed))


class QpackSection(ctypes.Structure):
    """osm_qpack_section_c: one entry of a qpack section table."""

    _fields_ = [("name", c_char_p), ("dtype", c_char_p), ("rank", c_uint32), ("rows", c_uint64),
                ("cols", c_uint64), ("offset", c_uint64), ("size", c_uint64)]


def qpack_expert_repack(g: Geometry, sections, slot_stride, slot=None):
    """sections: dicts with name, dtype, shape (rows, cols), offset, size.
    Returns (blob or None, identity)."""
    arr = (QpackSection * max(len(sections), 1))(*[
        QpackSection(s["name"].encode(), s["dtype"].encode(), len(s["shape"]), s["shape"][0],
                     s["shape"][1] if len(s["shape"]) > 1 else 0, s["offset"], s["size"]) for s in sections])
    ident = c_int(0)
    blob = None
    if slot is not None:
        sl = np.ascontiguousarray(slot).view(np.uint8)
        blob = np.zeros(expert_blob_bytes(g), np.uint8)
        check(load().osm_qpack_expert_repack(ctypes.byref(g), ctypes.cast(arr, c_void_p), len(sections), slot_stride,
                                             _p(sl), _p(blob), blob.size, ctypes.byref(ident)))
    else:
        check(load().osm_qpack_expert_repack(ctypes.byref(g), ctypes.cast(arr, c_void_p), len(sections), slot_stride,
                                             None, None, 0, ctypes.byref(ident)))
    return blob, bool(ident.value)


class QpackInfo(ctypes.Structure):
    """osm_qpack_info."""

    _fields_ = [("magic", c_char_p), ("model_name", c_char_p), ("source_checkpoint", c_char_p),
                ("version", c_uint32), ("expert_count", c_uint32), ("layer_count", c_uint32),
                ("section_count", c_uint32), ("expert_stride", c_uint64), ("quant_bits", ctypes.c_int32),
                ("quant_group_size", ctypes.c_int32)]


class QpackReader(_Handle):
    """QpackReader (container/qpack.hpp:15-90): the container's manifest and
    layout, parsed and checked on open; fixed-stride expert reads."""

    _destroy = "osm_qpack_close"

    def __init__(self, container_dir):
        h = c_void_p()
        check(load().osm_qpack_open(os.fsencode(container_dir), ctypes.byref(h)))
        super().__init__(h)
        info = QpackInfo()
        check(load().osm_qpack_get_info(self.h, ctypes.byref(info)))
        self.magic = info.magic.decode()
        self.model_name = info.model_name.decode()
        self.source_checkpoint = info.source_checkpoint.decode()
        self.version = info.version
        self.expert_count, self.layer_count = info.expert_count, info.layer_count
        self.expert_stride = info.expert_stride
        self.quant_bits = None if info.quant_bits < 0 else info.quant_bits
        self.quant_group_size = None if info.quant_group_size < 0 else info.quant_group_size
        self.sections = [self._section(i) for i in range(info.section_count)]
        lin = np.zeros(max(self.layer_count, 1), np.uint8)
        check(load().osm_qpack_linear_layers(self.h, _p(lin), lin.size))
        self.linear_layers = [bool(v) for v in lin[:self.layer_count]]

    def _section(self, i) -> dict:
        c = QpackSection()
        check(load().osm_qpack_get_section(self.h, i, ctypes.byref(c)))
        dims = c_uint32(0)
        check(load().osm_qpack_section_shape(self.h, i, None, 0, ctypes.byref(dims)))
        shape = np.zeros(max(dims.value, 1), np.uint64)
        check(load().osm_qpack_section_shape(self.h, i, _p(shape), dims.value, ctypes.byref(dims)))
        return {"name": c.name.decode(), "dtype": c.dtype.decode(), "shape": [int(v) for v in shape[:dims.value]],
                "offset": int(c.offset), "size": int(c.size)}

    def find_section(self, name):
        """QpackLayout::find_section: the entry, or None."""
        c = QpackSection()
        if load().osm_qpack_find_section(self.h, name.encode(), ctypes.byref(c)) != OSM_OK:
            return None
        return next(s for s in self.sections if s["name"] == name)

    def file_size(self, relative_path):
        """manifest.files[relative_path], or None when not declared."""
        v = c_uint64(0)
        if load().osm_qpack_file_size(self.h, os.fsencode(relative_path), ctypes.byref(v)) != OSM_OK:
            return None
        return int(v.value)

    def read_expert(self, layer, expert, destination_bytes=None) -> np.ndarray:
        n = self.expert_stride if destination_bytes is None else destination_bytes
        out = np.empty(n, np.uint8)
        check(load().osm_qpack_read_expert(self.h, layer, expert, _p(out), n))
        return out


class PreadStorage(_Handle):
    """PosixPreadExpertStorage: <container_dir>/packed_experts/layer_LL.bin
    holds layer LL's `experts` blobs back to back at `stride`."""

    _destroy = "osm_expert_storage_destroy"

    def __init__(self, container_dir, layers, experts, stride):
        h = c_void_p()
        check(load().osm_pread_storage_create(os.fsencode(container_dir), layers, experts, stride, ctypes.byref(h)))
        super().__init__(h)
        self.stride = stride

    @staticmethod
    def layer_path(container_dir, layer):
        return os.path.join(container_dir, "packed_experts", f"layer_{layer:02d}.bin")

    def read(self, layers, experts, dest_bytes=None) -> list:
        """Blobs of (layers[i], experts[i]), read in one call."""
        n = len(experts)
        size = self.stride if dest_bytes is None else dest_bytes
        outs = [np.empty(size, np.uint8) for _ in range(n)]
        ls, es = _c(layers, np.uint32), _c(experts, np.uint32)
        dests = (c_void_p * max(n, 1))(*[o.ctypes.data for o in outs])
        check(load().osm_expert_storage_read(self.h, _p(ls), _p(es), dests, n, size))
        return outs


class QpackStorage(PreadStorage):
    """QpackExpertStorage over a qpack container: whole expertStride slots,
    or, given a geometry, each slot repacked into that geometry's blob."""

    def __init__(self, container_dir, g: "Geometry | None" = None):
        h = c_void_p()
        check(load().osm_qpack_storage_create(os.fsencode(container_dir),
                                              ctypes.byref(g) if g is not None else None, ctypes.byref(h)))
        _Handle.__init__(self, h)
        self.stride = load().osm_expert_storage_stride(self.h)


class HostExpertCache(_Handle):
    """ExpertCache (host L1) over a Python storage callback, or over a
    native storage (from_storage)."""

    _destroy = "osm_host_cache_destroy"

    def __init__(self, stride, budget, read_fn, minimum_slots=1, pinned=False):
        def _cb(user, layers, experts, dests, count, stride_):
            try:
                ls = [layers[i] for i in range(count)]
                es = [experts[i] for i in range(count)]
                ds = [np.ctypeslib.as_array((ctypes.c_uint8 * stride_).from_address(dests[i])) for i in range(count)]
                return int(read_fn(ls, es, ds) or 0)
            except Exception:
                return 1

        self._cb = READ_EXPERTS_FN(_cb)
        h = c_void_p()
        check(load().osm_host_cache_create(stride, budget, minimum_slots, 1 if pinned else 0, self._cb, None, ctypes.byref(h)))
        super().__init__(h)
        self.stride = stride

    @classmethod
    def from_storage(cls, storage: "PreadStorage", budget, minimum_slots=1, pinned=False) -> "HostExpertCache":
        h = c_void_p()
        check(load().osm_host_cache_create_with_storage(storage.h, budget, minimum_slots, 1 if pinned else 0,
                                                        ctypes.byref(h)))
        obj = cls.__new__(cls)
        _Handle.__init__(obj, h)
        obj.stride = storage.stride
        obj._storage = storage  # the storage must outlive the cache
        return obj

    def fetch(self, layer, experts):
        e = _c(experts, np.uint32)
        slots = np.empty(e.size, np.uint64)
        ptrs = (c_void_p * max(e.size, 1))()
        check(load().osm_host_cache_fetch(self.h, layer, _p(e), e.size, _p(slots), ctypes.cast(ptrs, c_void_p)))
        blobs = [np.ctypeslib.as_array((ctypes.c_uint8 * self.stride).from_address(ptrs[i])).copy() for i in range(e.size)]
        return slots, blobs

    def resident_slot(self, layer, expert):
        s = load().osm_host_cache_resident_slot(self.h, layer, expert)
        return None if s < 0 else int(s)

    def stats(self) -> dict:
        st = HostCacheStats()
        load().osm_host_cache_stats_get(self.h, ctypes.byref(st))
        return {n: getattr(st, n) for n, _ in HostCacheStats._fields_}


class ExpertCache(_Handle):
    """VulkanResidentExpertCache counterpart: LFU+recency over one HBM slab."""

    _destroy = "osm_expert_cache_destroy"

    def __init__(self, ctx, budget, store: ExpertStore = None, host_cache: HostExpertCache = None, g: Geometry = None):
        h = c_void_p()
        if store is not None:
            check(load().osm_expert_cache_create_from_store(ctx.h, store.h, budget, ctypes.byref(h)))
            self.g = store.g
        else:
            check(load().osm_expert_cache_create_from_host_cache(ctx.h, host_cache.h, ctypes.byref(g), budget, ctypes.byref(h)))
            self.g = g
        super().__init__(h)
        ctx._adopt(self)
        self.ctx = ctx
        self._keep = (store, host_cache)

    def get(self, layer, expert) -> int:
        p = c_void_p()
        check(load().osm_expert_cache_get(self.h, layer, expert, ctypes.byref(p)))
        return p.value

    def run(self, layer, expert, x) -> np.ndarray:
        xv = _c(x, np.float32)
        out = np.empty(self.g.hidden, np.float32)
        check(load().osm_expert_cache_run(self.h, layer, expert, _p(xv), xv.size, _p(out), out.size))
        return out

    def contains(self, layer, expert) -> bool:
        return bool(load().osm_expert_cache_contains(self.h, layer, expert))

    def stats(self) -> dict:
        st = ExpertCacheStats()
        load().osm_expert_cache_stats_get(self.h, ctypes.byref(st))
        return {n: getattr(st, n) for n, _ in ExpertCacheStats._fields_}

    @property
    def bytes_filled(self) -> int:
        return load().osm_expert_cache_bytes_filled(self.h)


def run_cached_layers(ctx, layers, cache_layers, cache, x, picks=None) -> np.ndarray:
    """Chained sublayers through the capped cache in one native call. picks:
    None (route on the device) or (ids [n][tokens][k], weights [n][tokens][k])."""
    xv = _c(x, np.float32).reshape(-1, layers[0].g.hidden)
    hs = (c_void_p * len(layers))(*[m.h.value if isinstance(m.h, c_void_p) else m.h for m in layers])
    cl = _c(cache_layers, np.uint32)
    y = np.empty_like(xv)
    ids = w = None
    if picks is not None:
        ids, w = _c(picks[0], np.uint32), _c(picks[1], np.float32)
    check(load().osm_moe_run_cached_layers(ctx.h, ctypes.cast(hs, c_void_p), _p(cl), len(layers), cache.h, _p(xv),
                                           xv.shape[0], _p(ids) if ids is not None else None,
                                           _p(w) if w is not None else None, _p(y)))
    return y


class CachePolicy(_Handle):
    """The resident cache's LFU+recency policy alone (host only)."""

    _destroy = "osm_cache_policy_destroy"

    def __init__(self, budget):
        h = c_void_p()
        check(load().osm_cache_policy_create(budget, ctypes.byref(h)))
        super().__init__(h)

    def get(self, layer, expert, nbytes):
        ev = np.zeros(64, np.uint64)
        n = c_size_t(0)
        r = load().osm_cache_policy_get(self.h, layer, expert, nbytes, _p(ev), ev.size, ctypes.byref(n))
        if r < 0:
            raise OsmError(-r, last_error())
        return bool(r), [int(v) for v in ev[: n.value]]

    def contains(self, layer, expert) -> bool:
        return bool(load().osm_cache_policy_contains(self.h, layer, expert))

    def stats(self) -> dict:
        st = ExpertCacheStats()
        load().osm_cache_policy_stats_get(self.h, ctypes.byref(st))
        return {n: getattr(st, n) for n, _ in ExpertCacheStats._fields_}


# ---- synthetic inputs -----------------------------------------------------------------
def synth_expert_blob(ctx, seed, layer, expert, g: Geometry) -> np.ndarray:
    out = np.empty(expert_blob_bytes(g), np.uint8)
    check(load().osm_synth_expert_blob(ctx.h, seed, layer, expert, ctypes.byref(g), _p(out), out.size))
    return out


def synth_router_bf16(ctx, seed, layer, experts, hidden) -> np.ndarray:
    out = np.empty(experts * hidden, np.uint16)
    check(load().osm_synth_router_bf16(ctx.h, seed, layer, experts, hidden, _p(out)))
    return out


def synth_shared_gate_bf16(ctx, seed, layer, hidden) -> np.ndarray:
    out = np.empty(hidden, np.uint16)
    check(load().osm_synth_shared_gate_bf16(ctx.h, seed, layer, hidden, _p(out)))
    return out


def synth_norm_weight(ctx, seed, layer, hidden) -> np.ndarray:
    out = np.empty(hidden, np.float32)
    check(load().osm_synth_norm_weight(ctx.h, seed, layer, hidden, _p(out)))
    return out


def synth_tokens(ctx, seed, first_token, count, hidden) -> np.ndarray:
    out = np.empty(count * hidden, np.float32)
    check(load().osm_synth_tokens(ctx.h, seed, first_token, count, hidden, _p(out)))
    return out.reshape(count, hidden)


def synth_tokens_device(ctx, seed, first_token, count, hidden, dev_ptr):
    check(load().osm_synth_tokens_device(ctx.h, seed, first_token, count, hidden, dev_ptr))
