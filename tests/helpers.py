"""Fixture builders and metrics shared by the tests."""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

META_F32, META_F16, META_BF16 = 0, 1, 2


def pack_q4(q: np.ndarray) -> np.ndarray:
    """[rows, cols] nibbles 0..15 -> [rows, cols/8] uint32, low nibble first."""
    q = np.asarray(q, np.uint32)
    rows, cols = q.shape
    q = q.reshape(rows, cols // 8, 8)
    words = np.zeros((rows, cols // 8), np.uint32)
    for lane in range(8):
        words |= q[:, :, lane] << np.uint32(4 * lane)
    return words


def unpack_q4(words: np.ndarray) -> np.ndarray:
    w = np.asarray(words, np.uint32)
    lanes = [(w >> np.uint32(4 * j)) & np.uint32(0xF) for j in range(8)]
    return np.stack(lanes, axis=-1).reshape(*w.shape[:-1], w.shape[-1] * 8).astype(np.uint8)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def meta_encode(values: np.ndarray, meta: int) -> np.ndarray:
    v = np.ascontiguousarray(values, np.float32)
    if meta == META_F32:
        return v.view(np.uint8).ravel()
    if meta == META_F16:
        return v.astype(np.float16).view(np.uint8).ravel()
    return bf16_bits(v).view(np.uint8).ravel()


def meta_decode(values: np.ndarray, meta: int) -> np.ndarray:
    """The fp32 the device sees for metadata stored as `meta`."""
    v = np.ascontiguousarray(values, np.float32)
    if meta == META_F32:
        return v
    if meta == META_F16:
        return v.astype(np.float16).astype(np.float32)
    return bf16_to_f32(bf16_bits(v))


def make_blob(projections, meta: int) -> np.ndarray:
    """projections: three (packed u32 [out, in/8], scales [out, g], biases [out, g])
    in gate, up, down order -> the qpack-ordered expert blob."""
    parts = []
    for packed, s, b in projections:
        parts.append(np.ascontiguousarray(packed, np.uint32).view(np.uint8).ravel())
        parts.append(meta_encode(s, meta))
        parts.append(meta_encode(b, meta))
    return np.concatenate(parts)


def rel_l2(actual, expected) -> float:
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-30))


def max_abs(actual, expected) -> float:
    return float(np.max(np.abs(np.asarray(actual, np.float64) - np.asarray(expected, np.float64))))


# ---- fixtures restated from the reference's own tests --------------------------------
def gemv_fixture():
    """tests/vulkan_q4_gemv_test.cpp:27-115 (7 rows x 128 columns, group 64)."""
    out_dim, packed_cols, group = 7, 16, 64
    in_dim = packed_cols * 8
    q = np.zeros((out_dim, in_dim), np.uint32)
    for row in range(out_dim):
        for word in range(packed_cols):
            for lane in range(8):
                q[row, word * 8 + lane] = (row * 7 + word * 3 + lane * (word % 5 + 1)) & 0xF
    gpr = in_dim // group
    scales = np.zeros((out_dim, gpr), np.float32)
    biases = np.zeros((out_dim, gpr), np.float32)
    for row in range(out_dim):
        for g in range(gpr):
            scales[row, g] = np.float32(0.125) + np.float32(0.075) * np.float32(row + 2 * g + 1)
            biases[row, g] = (np.float32(-0.45) if g == 0 else np.float32(0.30)) + np.float32(0.035) * np.float32(row)
    x = np.array([np.float32((i % 17) - 8) * np.float32(0.0625) + np.float32((i * 7) % 5) * np.float32(0.0175)
                  for i in range(in_dim)], np.float32)
    return pack_q4(q), out_dim, packed_cols, scales, biases, group, x


def cache_fixture_expert(expert: int, meta: int = META_BF16):
    """The three-expert qpack of tests/vulkan_resident_expert_cache_test.cpp:51-132:
    hidden 128, intermediate 64, group 64, BF16 metadata."""
    def proj(seed, out_dim, packed_cols):
        in_dim = packed_cols * 8
        q = np.zeros((out_dim, in_dim), np.uint32)
        for row in range(out_dim):
            for word in range(packed_cols):
                for lane in range(8):
                    q[row, word * 8 + lane] = (seed * 3 + expert * 5 + row * 7 + word * 2 + lane) & 0xF
        gpr = in_dim // 64
        s = np.zeros((out_dim, gpr), np.float32)
        b = np.zeros((out_dim, gpr), np.float32)
        for row in range(out_dim):
            for g in range(gpr):
                s[row, g] = np.float32(((seed + expert + row + g) % 6) + 1) * np.float32(0.125)
                b[row, g] = np.float32(((seed * 2 + expert + row + g) % 7) - 3) * np.float32(0.125)
        return pack_q4(q), s, b

    return make_blob([proj(1, 64, 16), proj(2, 64, 16), proj(3, 128, 8)], meta)


def cache_fixture_token(seed: int) -> np.ndarray:
    """token() of tests/vulkan_resident_expert_cache_test.cpp:270-279."""
    return np.array([np.float32(((i * (seed + 5)) % 31) - 15) * np.float32(0.03125) for i in range(128)], np.float32)


def random_projection(rng, out_dim, in_dim, group, meta):
    """Seeded random q4 projection in the BASELINE distribution."""
    q = rng.integers(0, 16, size=(out_dim, in_dim), dtype=np.uint32)
    s = np.abs(rng.normal(0, 0.02, size=(out_dim, in_dim // group))).astype(np.float32)
    b = (-8.0 * meta_decode(s, meta) + rng.normal(0, 0.002, size=s.shape)).astype(np.float32)
    return pack_q4(q), meta_decode(s, meta), meta_decode(b, meta)


def random_blob(rng, hidden, inter, group, meta):
    projs = [random_projection(rng, inter, hidden, group, meta),
             random_projection(rng, inter, hidden, group, meta),
             random_projection(rng, hidden, inter, group, meta)]
    return make_blob(projs, meta), projs


def pmap(fn, items, workers=None):
    """fn over items on a thread pool (the oracle's C calls release the GIL);
    results in item order. At most 16 threads: the CPU share of one GPU."""
    items = list(items)
    n = workers or min(16, os.cpu_count() or 1, max(1, len(items)))
    with ThreadPoolExecutor(max_workers=n) as ex:
        return list(ex.map(fn, items))


def write_qpack(root, layer_slots, sections, stride, *, linear_layers=None, magic="QPACK", version=1,
                quant_bits=4, quant_group_size=None, layout_text=None, declare=True, model_name="qwen3_next"):
    """A qpack container (container/qpack.hpp:15-90) at `root`:
    packed_experts/layer_LL.bin from layer_slots[LL] (uint8 [experts, stride]),
    packed_experts/layout.json from `sections` (dicts with name, dtype,
    shape, offset, size) unless layout_text gives the file's text, and a
    manifest.json declaring every file with its size (declare=False leaves
    the layer files out). quant_group_size None writes null quantization."""
    import json
    pe = os.path.join(root, "packed_experts")
    os.makedirs(pe, exist_ok=True)
    layers = len(layer_slots)
    experts = layer_slots[0].shape[0] if layers else 0
    if layout_text is None:
        layout_text = json.dumps({
            "expertCount": experts, "layerCount": layers, "expertStride": stride,
            "sections": [{"name": s["name"], "dtype": s["dtype"], "shape": list(s["shape"]),
                          "offset": s["offset"], "size": s["size"]} for s in sections],
            "linearLayers": list(linear_layers) if linear_layers is not None else [True] * layers,
        }, indent=2)
    with open(os.path.join(pe, "layout.json"), "w") as f:
        f.write(layout_text)
    files = {"packed_experts/layout.json": os.path.getsize(os.path.join(pe, "layout.json"))}
    for l, slots in enumerate(layer_slots):
        path = os.path.join(pe, f"layer_{l:02d}.bin")
        np.ascontiguousarray(slots, dtype=np.uint8).tofile(path)
        if declare:
            files[f"packed_experts/layer_{l:02d}.bin"] = os.path.getsize(path)
    manifest = {"magic": magic, "version": version, "modelName": model_name,
                "sourceCheckpoint": "synthetic", "quantBits": quant_bits if quant_group_size else None,
                "quantGroupSize": quant_group_size, "files": files}
    with open(os.path.join(root, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=2)
    return root


def qpack_q4_sections(D, I, G, meta_dtype, order=None, gap=0, extra=()):
    """The nine sections of one q4 expert slot (gate/up/down x weight/scales/
    biases) in `order` (names; default the blob's), each followed by `gap`
    bytes; `extra` adds (name, dtype, shape, size) entries first. Returns
    (sections, slot stride)."""
    esz = 4 if meta_dtype == "F32" else 2
    shapes = {}
    for p in ("gate_proj", "up_proj", "down_proj"):
        out, inn = (I, D) if p != "down_proj" else (D, I)
        shapes[p + ".weight"] = ("U32", (out, inn // 8), out * inn // 8 * 4)
        shapes[p + ".scales"] = (meta_dtype, (out, inn // G), out * inn // G * esz)
        shapes[p + ".biases"] = (meta_dtype, (out, inn // G), out * inn // G * esz)
    for name, dt, shape, size in extra:
        shapes[name] = (dt, shape, size)
    names = [e[0] for e in extra] + (order or [p + s for p in ("gate_proj", "up_proj", "down_proj")
                                               for s in (".weight", ".scales", ".biases")])
    secs, off = [], 0
    for n in names:
        dt, shape, size = shapes[n]
        secs.append({"name": n, "dtype": dt, "shape": tuple(shape), "offset": off, "size": size})
        off += size + gap
    return secs, off


def blob_to_slot(blob, sections, stride, D, I, G, meta_dtype, fill=0xA5):
    """The q4 blob's nine sections placed at the table's offsets in a slot of
    `stride` bytes (the rest `fill`)."""
    esz = 4 if meta_dtype == "F32" else 2
    parts, off = {}, 0
    for p in ("gate_proj", "up_proj", "down_proj"):
        out, inn = (I, D) if p != "down_proj" else (D, I)
        for s, n in ((".weight", out * inn // 2), (".scales", out * inn // G * esz), (".biases", out * inn // G * esz)):
            parts[p + s] = blob[off:off + n]
            off += n
    slot = np.full(stride, fill, np.uint8)
    for s in sections:
        if s["name"] in parts:
            slot[s["offset"]:s["offset"] + s["size"]] = parts[s["name"]]
    return slot


def correlated_trace(rng, layers, steps, k, experts, repeat_p):
    """Routed experts per (step, layer), each [1, k] uint32: each of a layer's
    k picks repeats one of that layer's previous-step picks with probability
    repeat_p, else it is a fresh expert; picks within a step are distinct.
    The capped-cache workload of the 48-layer stack (p = 0.6)."""
    prev = [None] * layers
    trace = []
    for _s in range(steps):
        row = []
        for layer in range(layers):
            ids = []
            for _j in range(k):
                cands = [e for e in (prev[layer] or []) if e not in ids]
                if cands and rng.random() < repeat_p:
                    ids.append(int(rng.choice(cands)))
                    continue
                while True:
                    e = int(rng.integers(experts))
                    if e not in ids:
                        break
                ids.append(e)
            prev[layer] = ids
            row.append(np.array(ids, np.uint32).reshape(1, k))
        trace.append(row)
    return trace
