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
#include <cstdio>
#include <cstring>
#include <fstream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <system_error>

#include "json.hpp"
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

// ---- the container (container/qpack.cpp:41-247) ------------------------------
namespace {

json::Value read_json_file(const std::filesystem::path& path) {
  std::ifstream in(path, std::ios::binary);
  if (!in) throw std::runtime_error("qpack: unable to open JSON file: " + path.string());
  std::ostringstream text;
  text << in.rdbuf();
  try {
    return json::parse(text.str());
  } catch (const json::JsonError& e) {
    throw std::runtime_error("qpack: invalid JSON in " + path.string() + ": " + e.what());
  }
}

std::optional<std::uint32_t> optional_u32(const json::Value& obj, const char* key) {
  if (!obj.contains(key) || obj.at(key).is_null()) return std::nullopt;
  return obj.at(key).as_u32();
}

QpackManifest parse_manifest(const std::filesystem::path& path) {
  const json::Value j = read_json_file(path);
  QpackManifest out;
  try {
    out.magic = j.at("magic").as_string();
    out.version = j.at("version").as_u32();
    out.model_name = j.at("modelName").as_string();
    out.source_checkpoint = j.at("sourceCheckpoint").as_string();
    out.quant_bits = optional_u32(j, "quantBits");
    out.quant_group_size = optional_u32(j, "quantGroupSize");
    const json::Value& files = j.at("files");
    if (!files.is_object()) throw std::runtime_error("qpack: manifest.files must be an object");
    for (const auto& [name, size] : files.members) out.files.emplace(name, size.as_u64());
  } catch (const json::JsonError& e) {
    throw std::runtime_error("qpack: malformed manifest " + path.string() + ": " + e.what());
  }
  return out;
}

QpackLayout parse_layout(const std::filesystem::path& path) {
  const json::Value j = read_json_file(path);
  QpackLayout out;
  try {
    out.expert_count = j.at("expertCount").as_u32();
    out.layer_count = j.at("layerCount").as_u32();
    out.expert_stride = j.at("expertStride").as_u64();
    const json::Value& linear = j.at("linearLayers");
    if (!linear.is_array()) throw json::JsonError("linearLayers: type must be array");
    for (const auto& v : linear.items) out.linear_layers.push_back(v.as_bool());
    const json::Value& sections = j.at("sections");
    if (!sections.is_array()) throw std::runtime_error("qpack: layout.sections must be an array");
    out.sections.reserve(sections.items.size());
    for (const auto& item : sections.items) {
      QpackSection sec;
      sec.name = item.at("name").as_string();
      sec.dtype = item.at("dtype").as_string();
      const json::Value& shape = item.at("shape");
      if (!shape.is_array()) throw json::JsonError("shape: type must be array");
      for (const auto& d : shape.items) sec.shape.push_back(d.as_u64());
      sec.offset = item.at("offset").as_u64();
      sec.size = item.at("size").as_u64();
      out.sections.push_back(std::move(sec));
    }
  } catch (const json::JsonError& e) {
    throw std::runtime_error("qpack: malformed layout " + path.string() + ": " + e.what());
  }
  return out;
}

std::uint64_t file_size_of(const std::filesystem::path& path) {
  std::error_code ec;
  const auto n = std::filesystem::file_size(path, ec);
  if (ec) throw std::runtime_error("qpack: unable to stat " + path.string() + ": " + ec.message());
  return n;
}

void validate_declared_file(const std::filesystem::path& root, const QpackManifest& m, const std::string& rel) {
  const auto it = m.files.find(rel);
  if (it == m.files.end()) throw std::runtime_error("qpack: manifest does not declare required file: " + rel);
  if (file_size_of(root / rel) != it->second) throw std::runtime_error("qpack: file size disagrees with manifest: " + rel);
}

// Packed words x (32 / bits) and scale groups x group size must agree for
// each projection that has both sections (container/qpack.cpp:136-170).
void validate_expert_quantization(const QpackManifest& m, const QpackLayout& layout) {
  if (!m.quant_bits || !m.quant_group_size) return;
  const std::uint32_t bits = *m.quant_bits, group = *m.quant_group_size;
  if (bits == 0 || group == 0 || (32U % bits) != 0U) throw std::runtime_error("qpack: invalid expert quantization metadata");
  for (const char* prefix : {"gate_proj", "up_proj", "down_proj"}) {
    const QpackSection* w = layout.find_section(std::string(prefix) + ".weight");
    const QpackSection* sc = layout.find_section(std::string(prefix) + ".scales");
    if (w == nullptr || sc == nullptr) continue;
    if (w->shape.empty() || sc->shape.empty())
      throw std::runtime_error(std::string("qpack: quantized expert section has empty shape: ") + prefix);
    const std::uint64_t from_weight = w->shape.back() * (32U / bits);
    const std::uint64_t from_scales = sc->shape.back() * group;
    if (from_weight == 0 || from_weight != from_scales)
      throw std::runtime_error(std::string("qpack: expert quantization disagrees with packed shapes: ") + prefix);
  }
}

}  // namespace

const QpackSection* QpackLayout::find_section(std::string_view name) const noexcept {
  for (const auto& s : sections)
    if (s.name == name) return &s;
  return nullptr;
}

std::filesystem::path QpackReader::layer_path(std::uint32_t layer) const {
  return PosixPreadExpertStorage::layer_path(dir_, layer);
}

QpackReader::QpackReader(std::filesystem::path container_dir)
    : dir_(std::move(container_dir)),
      manifest_(parse_manifest(dir_ / "manifest.json")),
      layout_(parse_layout(dir_ / "packed_experts" / "layout.json")) {
  if (manifest_.magic != kMagic) throw std::runtime_error("qpack: unsupported magic: " + manifest_.magic);
  if (manifest_.version != kManifestVersion)
    throw std::runtime_error("qpack: unsupported manifest version: " + std::to_string(manifest_.version));
  if (layout_.layer_count == 0) throw std::runtime_error("qpack: layerCount must be non-zero");
  if (layout_.sections.empty()) throw std::runtime_error("qpack: sections must not be empty");
  if (layout_.linear_layers.size() != layout_.layer_count)
    throw std::runtime_error("qpack: linearLayers length must equal layerCount");
  for (const auto& s : layout_.sections) {
    if (s.name.empty() || s.size == 0) throw std::runtime_error("qpack: section name/size is invalid");
    if (s.offset > layout_.expert_stride || s.size > layout_.expert_stride - s.offset)
      throw std::runtime_error("qpack: section exceeds expertStride: " + s.name);
  }
  if (manifest_.quant_bits.has_value() != manifest_.quant_group_size.has_value())
    throw std::runtime_error("qpack: quantBits and quantGroupSize must both be present or both be null");
  validate_expert_quantization(manifest_, layout_);
  if (layout_.expert_count == 0 || layout_.expert_stride == 0)
    throw std::runtime_error("qpack: expertCount and expertStride must be non-zero");
  if (layout_.expert_stride > std::numeric_limits<std::uint64_t>::max() / layout_.expert_count)
    throw std::runtime_error("qpack: layer byte size overflows uint64");
  const std::uint64_t layer_bytes = layout_.expert_count * layout_.expert_stride;
  validate_declared_file(dir_, manifest_, "packed_experts/layout.json");
  for (std::uint32_t layer = 0; layer < layout_.layer_count; ++layer) {
    const auto path = layer_path(layer);
    if (!std::filesystem::exists(path)) throw std::runtime_error("qpack: missing expert layer file: " + path.string());
    if (file_size_of(path) != layer_bytes)
      throw std::runtime_error("qpack: expert layer has unexpected byte size: " + path.string());
    validate_declared_file(dir_, manifest_, std::filesystem::relative(path, dir_).generic_string());
  }
}

void QpackReader::read_expert(std::uint32_t layer, std::uint32_t expert, std::span<std::byte> destination) const {
  if (layer >= layout_.layer_count) throw std::out_of_range("qpack: layer index out of range");
  if (expert >= layout_.expert_count) throw std::out_of_range("qpack: expert index out of range");
  if (destination.size() < layout_.expert_stride)
    throw std::invalid_argument("qpack: destination is smaller than expertStride");
  std::ifstream in(layer_path(layer), std::ios::binary);
  if (!in) throw std::runtime_error("qpack: unable to open expert layer file");
  const std::uint64_t offset = static_cast<std::uint64_t>(expert) * layout_.expert_stride;
  if (offset > static_cast<std::uint64_t>(std::numeric_limits<std::streamoff>::max()))
    throw std::runtime_error("qpack: expert offset exceeds streamoff range");
  in.seekg(static_cast<std::streamoff>(offset), std::ios::beg);
  if (!in) throw std::runtime_error("qpack: seek to expert failed");
  in.read(reinterpret_cast<char*>(destination.data()), static_cast<std::streamsize>(layout_.expert_stride));
  if (in.gcount() != static_cast<std::streamsize>(layout_.expert_stride))
    throw std::runtime_error("qpack: short expert read");
}

// ---- expert storage over the container -----------------------------------------
QpackExpertStorage::QpackExpertStorage(std::filesystem::path container_dir, const osm_expert_geometry* g)
    : reader_(std::move(container_dir)) {
  const QpackLayout& l = reader_.layout();
  if (l.expert_stride > static_cast<std::uint64_t>(std::numeric_limits<std::size_t>::max()))
    throw std::runtime_error("qpack: expertStride exceeds the address range");
  if (g != nullptr) {
    // The section table as plan_qpack_expert reads it: rank-2 shapes as
    // rows x columns.
    std::vector<QpackSectionView> views;
    views.reserve(l.sections.size());
    for (const auto& s : l.sections) {
      QpackSectionView v;
      v.name = s.name;
      v.dtype = s.dtype;
      v.rank = static_cast<std::uint32_t>(s.shape.size());
      v.rows = s.shape.size() > 0 ? s.shape[0] : 0U;
      v.cols = s.shape.size() > 1 ? s.shape[1] : 0U;
      v.offset = s.offset;
      v.size = s.size;
      views.push_back(v);
    }
    plan_ = plan_qpack_expert(views, l.expert_stride, *g);
  }
  pread_ = std::make_unique<PosixPreadExpertStorage>(reader_.container_dir(), l.layer_count, l.expert_count,
                                                     static_cast<std::size_t>(l.expert_stride));
}

std::size_t QpackExpertStorage::expert_stride_bytes() const noexcept {
  return plan_ ? plan_->blob_bytes : static_cast<std::size_t>(reader_.layout().expert_stride);
}

void QpackExpertStorage::read_experts(std::span<ExpertReadRequest> requests) {
  const std::size_t stride = expert_stride_bytes();
  for (const auto& r : requests)
    if (r.destination.size() < stride)
      throw std::invalid_argument("qpack expert storage: destination smaller than expert stride");
  const std::size_t slot = static_cast<std::size_t>(reader_.layout().expert_stride);
  if (!plan_ || (plan_->identity && slot <= stride)) {
    pread_->read_experts(requests);
    return;
  }
  // Whole slots into staging, then each slot's sections into its blob.
  std::vector<std::byte> staging(requests.size() * slot);
  std::vector<ExpertReadRequest> reads(requests.begin(), requests.end());
  for (std::size_t i = 0; i < reads.size(); ++i) reads[i].destination = std::span<std::byte>(staging.data() + i * slot, slot);
  pread_->read_experts(reads);
  for (std::size_t i = 0; i < requests.size(); ++i)
    repack_qpack_expert(*plan_, staging.data() + i * slot, requests[i].destination.data());
}

}  // namespace osm
