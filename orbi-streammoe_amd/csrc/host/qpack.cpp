// qpack.cpp -- an expert's qpack cache slot bound by section name.
//
// bind_qpack_q4_projection (backend/vulkan_qpack_expert.cpp:149-239) finds
// "<projection>.weight/.scales/.biases" in the container's section table by
// name and checks dtypes, ranks, shapes and byte ranges before reading. The
// same checks run here for gate_proj, up_proj and down_proj against the
// expert geometry, and the nine sections are then copied into the blob's
// canonical order (gate, up, down; packed, scales, biases each). The official
// layout already is that order, contiguous from offset 0
// (docs/OSM-39B-QPACK-EXPERT-GEOMETRY.md:35-42), so its slot is the blob as
// it stands. Unlike the reference, which widens scales and biases to fp32,
// the blob keeps them in their stored dtype, which must be the geometry's.
#include <cstring>
#include <stdexcept>

#include "osm_hip.hpp"

namespace osm {

namespace {

const char* meta_name(std::uint32_t dtype) {
  return dtype == OSM_META_F32 ? "F32" : dtype == OSM_META_F16 ? "F16" : "BF16";
}

}  // namespace

QpackExpertPlan plan_qpack_expert(std::span<const QpackSectionView> sections, std::uint64_t slot_stride,
                                  const osm_expert_geometry& g) {
  std::string d;
  if (!check_expert_geometry(g, &d)) throw std::invalid_argument(d);
  const osm_expert_offsets canon = osm_expert_layout(g);
  const std::size_t esz = osm_meta_bytes(g.meta_dtype);
  struct Proj {
    const char* name;
    std::uint64_t out, in;
    std::size_t q, s, b;
  };
  const Proj projs[3] = {{"gate_proj", g.inter, g.hidden, canon.gate_q, canon.gate_s, canon.gate_b},
                         {"up_proj", g.inter, g.hidden, canon.up_q, canon.up_s, canon.up_b},
                         {"down_proj", g.hidden, g.inter, canon.down_q, canon.down_s, canon.down_b}};
  auto find = [&](const std::string& name) -> const QpackSectionView* {
    for (const auto& s : sections)
      if (s.name == name) return &s;
    return nullptr;
  };
  QpackExpertPlan plan;
  plan.identity = true;
  std::size_t k = 0;
  for (const Proj& p : projs) {
    const std::string prefix(p.name);
    const auto* w = find(prefix + ".weight");
    const auto* sc = find(prefix + ".scales");
    const auto* bi = find(prefix + ".biases");
    if (!w || !sc || !bi) throw std::runtime_error("qpack expert: weight/scales/biases section set is incomplete");
    if (w->dtype != "U32") throw std::runtime_error("qpack expert: Q4 weight dtype must be U32");
    if (sc->dtype != bi->dtype) throw std::runtime_error("qpack expert: scale/bias dtypes must match");
    if (sc->dtype != "F32" && sc->dtype != "F16" && sc->dtype != "BF16")
      throw std::runtime_error("qpack expert: scale/bias dtype must be F32, F16, or BF16");
    if (sc->dtype != meta_name(g.meta_dtype))
      throw std::invalid_argument("qpack expert: scale/bias dtype differs from the expert geometry's");
    if (w->rank != 2 || sc->rank != 2 || bi->rank != 2)
      throw std::runtime_error("qpack expert: projection sections must be rank-2");
    const std::uint64_t groups = p.in / g.group;
    if (w->rows != p.out || w->cols * 8U != p.in || sc->rows != p.out || sc->cols != groups || bi->rows != p.out ||
        bi->cols != groups)
      throw std::runtime_error("qpack expert: " + prefix + " shapes disagree with the expert geometry");
    const std::uint64_t want[3] = {p.out * w->cols * 4U, p.out * groups * esz, p.out * groups * esz};
    const QpackSectionView* secs[3] = {w, sc, bi};
    const std::size_t dst[3] = {p.q, p.s, p.b};
    for (int i = 0; i < 3; ++i) {
      const auto& s = *secs[i];
      const std::uint64_t align = i == 0 ? 4U : esz;  // typed_section's alignment check
      if (s.size != want[i]) throw std::runtime_error("qpack expert: " + std::string(s.name) + " byte size disagrees with its shape");
      if (s.offset % align != 0U) throw std::runtime_error("qpack expert: misaligned " + std::string(s.name) + " section");
      if (s.offset > slot_stride || s.size > slot_stride - s.offset)
        throw std::runtime_error("qpack expert: " + std::string(s.name) + " section exceeds the slot");
      plan.src[k] = s.offset;
      plan.dst[k] = dst[i];
      plan.bytes[k] = static_cast<std::size_t>(s.size);
      plan.identity = plan.identity && s.offset == dst[i];
      ++k;
    }
  }
  plan.blob_bytes = canon.total;
  return plan;
}

void repack_qpack_expert(const QpackExpertPlan& plan, const std::byte* slot, std::byte* blob) {
  for (std::size_t k = 0; k < plan.src.size(); ++k) std::memcpy(blob + plan.dst[k], slot + plan.src[k], plan.bytes[k]);
}

}  // namespace osm
