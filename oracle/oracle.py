"""ctypes binding of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Loads oracle/_build/libosm_oracle.so -- this repository's restatement of the
reference CPU path -- and, when built, oracle/_ref/libosm_ref.so -- the
reference's own CPU sources compiled where they lie. Only tests/, the smoke()
check and bench.py's cpu_baseline leg use this module; the product never does.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int64, c_size_t, c_uint16, c_uint32, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "_build", "libosm_oracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libosm_ref.so")

META_F32, META_F16, META_BF16 = 0, 1, 2


class OracleError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"oracle code {code}: {msg}")
        self.code = code
        self.msg = msg


_P = c_void_p
_ORACLE_PROTOS = {
    "oracle_last_error": (c_char_p, []),
    "oracle_dequantize_affine_rows": (c_int, [_P, c_size_t, c_size_t, c_size_t, _P, c_size_t, _P, c_size_t, c_uint32, c_uint32, _P]),
    "oracle_quantize_affine_q4_rows": (c_int, [_P, c_size_t, c_size_t, c_size_t, c_size_t, _P, _P, _P, POINTER(c_float), POINTER(c_double)]),
    "oracle_matvec_row_major": (c_int, [_P, c_size_t, c_size_t, c_size_t, _P, c_size_t, _P]),
    "oracle_rms_norm_inplace": (c_int, [_P, c_size_t, c_size_t, c_size_t, _P, c_size_t, c_float]),
    "oracle_softmax_inplace": (c_int, [_P, c_size_t]),
    "oracle_route_top_k": (c_int, [_P, c_size_t, c_size_t, c_int, _P, _P]),
    "oracle_sigmoid": (c_float, [c_float]),
    "oracle_silu": (c_float, [c_float]),
    "oracle_swiglu_inplace": (c_int, [_P, c_size_t, _P, c_size_t]),
    "oracle_route_qwen_top_k": (c_int, [_P, c_size_t, _P, c_size_t, c_size_t, c_size_t, c_size_t, c_int, _P, _P, _P, _P]),
    "oracle_run_shared_expert": (c_int, [_P, c_size_t, _P, c_size_t, _P, c_size_t, _P, c_size_t, _P, c_size_t, c_size_t, c_size_t, _P, _P]),
    "oracle_bf16_to_float": (c_float, [c_uint16]),
    "oracle_libm_expf_checksums": (c_int, [c_uint32, c_uint64, c_uint32, _P]),
    "oracle_moe_sublayer_picks": (c_int, [_P, _P, c_float, _P, c_uint32, _P, _P, _P, c_uint32, c_uint32, c_uint32, c_int, _P]),
    "oracle_f16_to_float": (c_float, [c_uint16]),
    "oracle_expert_blob_bytes": (c_size_t, [c_uint32, c_uint32, c_uint32, c_int]),
    "oracle_expert_forward": (c_int, [_P, c_uint32, c_uint32, c_uint32, c_int, _P, _P]),
    "oracle_q4_gemv": (c_int, [_P, c_size_t, c_size_t, _P, _P, c_size_t, _P, _P]),
    "oracle_qwen_sparse_moe": (c_int, [_P, _P, c_uint32, c_uint32, c_int, _P, _P, _P, c_uint32, c_uint32, c_uint32, c_int, _P, _P, _P, _P, _P, _P]),
    "oracle_moe_sublayer": (c_int, [_P, _P, c_float, _P, c_uint32, c_uint32, c_int, _P, _P, _P, c_uint32, c_uint32, c_uint32, c_int, _P, _P, _P, _P, _P]),
    "oracle_synth_stream": (c_uint64, [c_uint64, c_uint32, c_uint32, c_uint32]),
    "oracle_synth_normal": (c_float, [c_uint64, c_uint64]),
    "oracle_synth_expert_blob": (None, [c_uint64, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_int, _P]),
    "oracle_synth_router_bf16": (None, [c_uint64, c_uint32, c_uint32, c_uint32, _P]),
    "oracle_synth_shared_gate_bf16": (None, [c_uint64, c_uint32, c_uint32, _P]),
    "oracle_synth_norm_weight": (None, [c_uint64, c_uint32, c_uint32, _P]),
    "oracle_synth_tokens": (None, [c_uint64, c_uint32, c_uint32, c_uint32, _P]),
    "oracle_host_cache_create": (_P, [c_size_t, c_size_t, c_size_t]),
    "oracle_host_cache_destroy": (None, [_P]),
    "oracle_host_cache_fetch": (c_int, [_P, c_uint32, _P, c_size_t, c_int, _P, POINTER(c_int)]),
    "oracle_host_cache_resident_slot": (c_int64, [_P, c_uint32, c_uint32]),
    "oracle_host_cache_stats": (None, [_P, _P]),
    "oracle_host_cache_storage_batches": (c_uint64, [_P]),
    "oracle_device_cache_create": (_P, [c_size_t]),
    "oracle_device_cache_destroy": (None, [_P]),
    "oracle_device_cache_get": (c_int, [_P, c_uint32, c_uint32, c_size_t, _P, c_size_t, POINTER(c_size_t)]),
    "oracle_device_cache_contains": (c_int, [_P, c_uint32, c_uint32]),
    "oracle_device_cache_stats": (None, [_P, _P]),
}

_REF_PROTOS = {
    "ref_last_error": (c_char_p, []),
    "ref_dequantize_affine_rows": (c_int, [_P, c_size_t, c_size_t, c_size_t, _P, c_size_t, _P, c_size_t, c_uint32, c_uint32, _P]),
    "ref_matvec_row_major": (c_int, [_P, c_size_t, c_size_t, c_size_t, _P, c_size_t, _P]),
    "ref_rms_norm_inplace": (c_int, [_P, c_size_t, c_size_t, c_size_t, _P, c_size_t, c_float]),
    "ref_route_top_k": (c_int, [_P, c_size_t, c_size_t, c_int, _P, _P]),
    "ref_swiglu_inplace": (c_int, [_P, c_size_t, _P]),
    "ref_route_qwen_top_k": (c_int, [_P, c_size_t, _P, c_size_t, c_size_t, c_size_t, c_size_t, c_int, _P, _P, _P, _P]),
    "ref_run_shared_expert": (c_int, [_P, c_size_t, _P, _P, _P, _P, c_size_t, _P, _P]),
    "ref_sparse_moe": (c_int, [_P, _P, c_uint32, c_uint32, _P, _P, _P, c_uint32, c_uint32, c_uint32, _P, _P, _P]),
    "ref_host_cache_create": (_P, [c_size_t, c_size_t, c_size_t]),
    "ref_host_cache_destroy": (None, [_P]),
    "ref_host_cache_fetch": (c_int, [_P, c_uint32, _P, c_size_t, c_int, _P]),
    "ref_host_cache_resident_slot": (c_int64, [_P, c_uint32, c_uint32]),
    "ref_host_cache_stats": (None, [_P, _P]),
    "ref_host_cache_storage_batches": (c_uint64, [_P]),
}


def _load(path, protos):
    lib = ctypes.CDLL(path)
    for name, (res, args) in protos.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_oracle = None
_ref = None


def lib():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_LIB):
            raise OracleError(-1, f"{ORACLE_LIB} not built (make -C oracle)")
        _oracle = _load(ORACLE_LIB, _ORACLE_PROTOS)
    return _oracle


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise OracleError(-1, f"{REF_LIB} not built (needs the reference checkout)")
        _ref = _load(REF_LIB, _REF_PROTOS)
    return _ref


def p(a):
    return c_void_p(a.ctypes.data) if a is not None else None


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def _check(rc, which="oracle"):
    if rc != 0:
        msg = (lib().oracle_last_error() if which == "oracle" else ref().ref_last_error()).decode()
        raise OracleError(rc, msg)


# ---- restated reference functions -------------------------------------------------------
def dequantize_affine_rows(packed, rows, packed_cols, scales, biases, bits=4, group_size=64, impl="oracle"):
    pk, s, b = u32(packed), f32(scales), f32(biases)
    per_word = 32 // bits if bits in (4, 8) else 1
    out = np.zeros(max(rows * packed_cols * per_word, 1), np.float32)
    fn = lib().oracle_dequantize_affine_rows if impl == "oracle" else ref().ref_dequantize_affine_rows
    _check(fn(p(pk), pk.size, rows, packed_cols, p(s), s.size, p(b), b.size, bits, group_size, p(out)), impl)
    return out


def quantize_affine_q4_rows(values, rows, cols, group):
    """single_expert_pilot.cpp:276-358: (packed, scales, biases, max_err, mean_err)."""
    v = f32(values).reshape(-1)
    packed = np.zeros(rows * (cols // 8) if cols % 8 == 0 else 1, np.uint32)
    groups = cols // group if group and cols % group == 0 else 1
    scales = np.zeros(max(rows * groups, 1), np.float32)
    biases = np.zeros_like(scales)
    mx = c_float(0)
    mean = c_double(0)
    _check(lib().oracle_quantize_affine_q4_rows(p(v), v.size, rows, cols, group, p(packed), p(scales), p(biases),
                                                ctypes.byref(mx), ctypes.byref(mean)))
    return packed, scales, biases, mx.value, mean.value


def matvec_row_major(weight, out_dim, in_dim, x, impl="oracle"):
    w, xv = f32(weight), f32(x)
    out = np.zeros(max(out_dim, 1), np.float32)
    fn = lib().oracle_matvec_row_major if impl == "oracle" else ref().ref_matvec_row_major
    _check(fn(p(w), w.size, out_dim, in_dim, p(xv), xv.size, p(out)), impl)
    return out


def rms_norm(values, rows, dim, weight, eps, impl="oracle"):
    v = f32(values).copy()
    w = f32(weight) if weight is not None else np.zeros(0, np.float32)
    fn = lib().oracle_rms_norm_inplace if impl == "oracle" else ref().ref_rms_norm_inplace
    _check(fn(p(v), v.size, rows, dim, p(w) if w.size else None, w.size, eps), impl)
    return v


def softmax(values):
    v = f32(values).copy()
    _check(lib().oracle_softmax_inplace(p(v), v.size))
    return v


def route_top_k(logits, k, normalize, impl="oracle"):
    lg = f32(logits)
    ids = np.zeros(k, np.uint32)
    pr = np.zeros(k, np.float32)
    fn = lib().oracle_route_top_k if impl == "oracle" else ref().ref_route_top_k
    _check(fn(p(lg), lg.size, k, 1 if normalize else 0, p(ids), p(pr)), impl)
    return ids, pr


def sigmoid(v):
    return lib().oracle_sigmoid(v)


def silu(v):
    return lib().oracle_silu(v)


def swiglu(gate, up, impl="oracle"):
    g, u = f32(gate).copy(), f32(up)
    if impl == "oracle":
        _check(lib().oracle_swiglu_inplace(p(g), g.size, p(u), u.size))
    else:
        _check(ref().ref_swiglu_inplace(p(g), g.size, p(u)), impl)
    return g


def route_qwen_top_k(hidden, router_weight, hidden_size, expert_count, top_k, norm_topk_prob=True, impl="oracle"):
    h, w = f32(hidden), f32(router_weight)
    logits = np.zeros(expert_count, np.float32)
    ids = np.zeros(top_k, np.uint32)
    wts = np.zeros(top_k, np.float32)
    mass = np.zeros(1, np.float32)
    fn = lib().oracle_route_qwen_top_k if impl == "oracle" else ref().ref_route_qwen_top_k
    _check(fn(p(h), h.size, p(w), w.size, hidden_size, expert_count, top_k, 1 if norm_topk_prob else 0, p(logits), p(ids), p(wts), p(mass)), impl)
    return {"logits": logits, "ids": ids, "weights": wts, "mass": float(mass[0])}


def run_shared_expert(hidden, gate, up, down, scalar_gate, hidden_size, inter, impl="oracle"):
    h, g, u, d, s = f32(hidden), f32(gate), f32(up), f32(down), f32(scalar_gate)
    out = np.zeros(hidden_size, np.float32)
    sg = np.zeros(1, np.float32)
    if impl == "oracle":
        _check(lib().oracle_run_shared_expert(p(h), h.size, p(g), g.size, p(u), u.size, p(d), d.size, p(s), s.size, hidden_size, inter, p(out), p(sg)))
    else:
        _check(ref().ref_run_shared_expert(p(h), hidden_size, p(g), p(u), p(d), p(s), inter, p(out), p(sg)), impl)
    return out, float(sg[0])


def bf16_to_float(bits):
    return lib().oracle_bf16_to_float(bits)


def libm_expf_checksums(first_bits, count, block):
    """Block checksums of the host libm's expf (std::exp of a float, as the
    reference's softmax calls it) over float bit patterns first_bits ..
    first_bits + count - 1: sum over each block's inputs i of
    bits(exp(x)) * (2 i + 1) mod 2^64."""
    out = np.zeros((count + block - 1) // block, np.uint64)
    _check(lib().oracle_libm_expf_checksums(first_bits, count, block, p(out)))
    return out


def f16_to_float(bits):
    return lib().oracle_f16_to_float(bits)


def expert_blob_bytes(hidden, inter, group=64, meta=META_BF16):
    return lib().oracle_expert_blob_bytes(hidden, inter, group, meta)


def expert_forward(blob, hidden, inter, group, meta, x):
    bl = np.ascontiguousarray(blob).view(np.uint8)
    xv = f32(x)
    out = np.zeros(hidden, np.float32)
    _check(lib().oracle_expert_forward(p(bl), hidden, inter, group, meta, p(xv), p(out)))
    return out


def q4_gemv(packed, out_dim, packed_cols, scales, biases, group_size, x):
    pk, s, b, xv = u32(packed), f32(scales), f32(biases), f32(x)
    y = np.zeros(out_dim, np.float32)
    _check(lib().oracle_q4_gemv(p(pk), out_dim, packed_cols, p(s), p(b), group_size, p(xv), p(y)))
    return y


def _ptr_table(blobs):
    arr = (c_void_p * len(blobs))(*[b.ctypes.data for b in blobs])
    return arr


def qwen_sparse_moe(hidden, router_f32, expert_blobs, shared_blob, shared_scalar_gate, hidden_size, inter, group, meta, top_k, norm_topk_prob=True):
    """One token: routing + weighted routed sum + gated shared expert."""
    h, r = f32(hidden), f32(router_f32)
    E = len(expert_blobs)
    table = _ptr_table(expert_blobs)
    sg = f32(shared_scalar_gate) if shared_scalar_gate is not None else None
    out = np.zeros(hidden_size, np.float32)
    ids = np.zeros(top_k, np.uint32)
    w = np.zeros(top_k, np.float32)
    mass = np.zeros(1, np.float32)
    sgo = np.zeros(1, np.float32)
    logits = np.zeros(E, np.float32)
    _check(lib().oracle_qwen_sparse_moe(p(h), p(r), E, top_k, 1 if norm_topk_prob else 0, ctypes.cast(table, c_void_p),
                                        p(shared_blob) if shared_blob is not None else None, p(sg),
                                        hidden_size, inter, group, meta, p(out), p(ids), p(w), p(mass), p(sgo), p(logits)))
    return {"out": out, "ids": ids, "weights": w, "mass": float(mass[0]), "shared_gate": float(sgo[0]), "logits": logits}


def moe_sublayer(residual, norm_weight, eps, router_f32, expert_blobs, shared_blob, shared_scalar_gate, hidden_size, inter, group, meta, top_k, norm_topk_prob=True):
    x, nw, r = f32(residual), f32(norm_weight), f32(router_f32)
    E = len(expert_blobs)
    table = _ptr_table(expert_blobs)
    sg = f32(shared_scalar_gate) if shared_scalar_gate is not None else None
    normalized = np.zeros(hidden_size, np.float32)
    out = np.zeros(hidden_size, np.float32)
    ids = np.zeros(top_k, np.uint32)
    w = np.zeros(top_k, np.float32)
    sgo = np.zeros(1, np.float32)
    _check(lib().oracle_moe_sublayer(p(x), p(nw), eps, p(r), E, top_k, 1 if norm_topk_prob else 0, ctypes.cast(table, c_void_p),
                                     p(shared_blob) if shared_blob is not None else None, p(sg),
                                     hidden_size, inter, group, meta, p(normalized), p(out), p(ids), p(w), p(sgo)))
    return {"out": out, "normalized": normalized, "ids": ids, "weights": w, "shared_gate": float(sgo[0])}


def moe_sublayer_picks(residual, norm_weight, eps, weights, pick_blobs, shared_blob, shared_scalar_gate, hidden_size, inter, group, meta):
    """The sublayer with given routed experts (no router): RMSNorm, pick i's
    expert blob accumulated with weights[i] in pick order, the sigmoid-gated
    shared expert, the residual."""
    x, nw, w = f32(residual), f32(norm_weight), f32(weights)
    table = _ptr_table(pick_blobs)
    sg = f32(shared_scalar_gate) if shared_scalar_gate is not None else None
    out = np.zeros(hidden_size, np.float32)
    _check(lib().oracle_moe_sublayer_picks(p(x), p(nw), eps, p(w), len(pick_blobs), ctypes.cast(table, c_void_p),
                                           p(shared_blob) if shared_blob is not None else None, p(sg),
                                           hidden_size, inter, group, meta, p(out)))
    return out


# ---- synthetic generator ----------------------------------------------------------------
def synth_expert_blob(seed, layer, expert, hidden, inter, group=64, meta=META_BF16):
    out = np.zeros(expert_blob_bytes(hidden, inter, group, meta), np.uint8)
    lib().oracle_synth_expert_blob(seed, layer, expert, hidden, inter, group, meta, p(out))
    return out


def synth_router_bf16(seed, layer, experts, hidden):
    out = np.zeros(experts * hidden, np.uint16)
    lib().oracle_synth_router_bf16(seed, layer, experts, hidden, p(out))
    return out


def synth_shared_gate_bf16(seed, layer, hidden):
    out = np.zeros(hidden, np.uint16)
    lib().oracle_synth_shared_gate_bf16(seed, layer, hidden, p(out))
    return out


def synth_norm_weight(seed, layer, hidden):
    out = np.zeros(hidden, np.float32)
    lib().oracle_synth_norm_weight(seed, layer, hidden, p(out))
    return out


def synth_tokens(seed, first_token, count, hidden):
    out = np.zeros(count * hidden, np.float32)
    lib().oracle_synth_tokens(seed, first_token, count, hidden, p(out))
    return out.reshape(count, hidden)


def bf16_bits_to_f32(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


SHARED_EXPERT_ID = 0xFFFFFFFF


def blob_sections(blob, hidden, inter, group=64, meta=META_BF16):
    """Splits a blob into its nine sections (gate/up/down x packed/scales/biases),
    metadata widened to fp32 (vulkan_qpack_expert.cpp:54-145)."""
    bl = np.ascontiguousarray(blob).view(np.uint8)
    ms = 4 if meta == META_F32 else 2
    off = 0
    out = []
    for out_dim, in_dim in ((inter, hidden), (inter, hidden), (hidden, inter)):
        nq = out_dim * in_dim // 8
        q = bl[off: off + nq * 4].view(np.uint32).reshape(out_dim, in_dim // 8)
        off += nq * 4
        ng = out_dim * (in_dim // group)
        metas = []
        for _ in range(2):
            raw = bl[off: off + ng * ms]
            off += ng * ms
            if meta == META_F32:
                v = raw.view(np.float32)
            elif meta == META_BF16:
                v = bf16_bits_to_f32(raw.view(np.uint16))
            else:
                v = raw.view(np.float16).astype(np.float32)
            metas.append(v.reshape(out_dim, in_dim // group).astype(np.float32))
        out.append((q, metas[0], metas[1]))
    return out


# ---- caches -------------------------------------------------------------------------------
class HostCache:
    """Restated host L1 cache over the pattern storage (impl 'oracle'), or the
    reference's own ExpertCache over the same storage (impl 'ref')."""

    def __init__(self, stride, budget, minimum_slots=1, impl="oracle"):
        self.impl = impl
        self.stride = stride
        if impl == "oracle":
            self.h = lib().oracle_host_cache_create(stride, budget, minimum_slots)
            if not self.h:
                raise OracleError(1, lib().oracle_last_error().decode())
        else:
            self.h = ref().ref_host_cache_create(stride, budget, minimum_slots)
            if not self.h:
                raise OracleError(1, ref().ref_last_error().decode())

    def fetch(self, layer, experts, fail_read=False):
        e = u32(experts)
        slots = np.zeros(max(e.size, 1), np.uint64)
        if self.impl == "oracle":
            ok = c_int(1)
            rc = lib().oracle_host_cache_fetch(self.h, layer, p(e), e.size, 1 if fail_read else 0, p(slots), ctypes.byref(ok))
            _check(rc)
            return [int(s) for s in slots[: e.size]], bool(ok.value)
        rc = ref().ref_host_cache_fetch(self.h, layer, p(e), e.size, 1 if fail_read else 0, p(slots))
        _check(rc, "ref")
        return [int(s) for s in slots[: e.size]], True

    def resident_slot(self, layer, expert):
        fn = lib().oracle_host_cache_resident_slot if self.impl == "oracle" else ref().ref_host_cache_resident_slot
        s = fn(self.h, layer, expert)
        return None if s < 0 else int(s)

    def stats(self):
        o = np.zeros(6, np.uint64)
        (lib().oracle_host_cache_stats if self.impl == "oracle" else ref().ref_host_cache_stats)(self.h, p(o))
        return dict(zip(("hits", "misses", "allocated_slots", "capacity_slots", "logical_bytes", "budget_bytes"), map(int, o)))

    def storage_batches(self):
        fn = lib().oracle_host_cache_storage_batches if self.impl == "oracle" else ref().ref_host_cache_storage_batches
        return int(fn(self.h))

    def __del__(self):
        try:
            if self.h:
                (lib().oracle_host_cache_destroy if self.impl == "oracle" else ref().ref_host_cache_destroy)(self.h)
        except Exception:
            pass


class DeviceCachePolicy:
    """Restated resident-cache policy (vulkan_resident_expert_cache.cpp:44-188)."""

    def __init__(self, budget):
        self.h = lib().oracle_device_cache_create(budget)
        if not self.h:
            raise OracleError(1, lib().oracle_last_error().decode())

    def get(self, layer, expert, nbytes):
        ev = np.zeros(64, np.uint64)
        n = c_size_t(0)
        rc = lib().oracle_device_cache_get(self.h, layer, expert, nbytes, p(ev), ev.size, ctypes.byref(n))
        if rc < 0:
            raise OracleError(rc, lib().oracle_last_error().decode())
        return bool(rc == 1), [int(v) for v in ev[: n.value]]

    def contains(self, layer, expert):
        return bool(lib().oracle_device_cache_contains(self.h, layer, expert))

    def stats(self):
        o = np.zeros(7, np.uint64)
        lib().oracle_device_cache_stats(self.h, p(o))
        return dict(zip(("hits", "misses", "loads", "evictions", "resident_entries", "resident_bytes", "budget_bytes"), map(int, o)))

    def __del__(self):
        try:
            if self.h:
                lib().oracle_device_cache_destroy(self.h)
        except Exception:
            pass
