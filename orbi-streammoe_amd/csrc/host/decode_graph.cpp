// decode_graph.cpp -- a decode step over a stack of MoE layers, and HIP
// graphs that capture such steps (or any enqueue-only sequence) for replay.
#include <string>
#include <utility>

#include "host_util.hpp"
#include "osm_hip.hpp"

namespace osm {

HipDispatchResult enqueue_decode_step(HipComputeContext& context, const HipDecodeStep& step) noexcept {
  HipDispatchResult r;
  const std::size_t n = step.layers.size();
  if (n == 0 || step.tables.size() != n || step.x == nullptr || step.y == nullptr) {
    r.diagnostic = "decode step needs layers, one expert table per layer, input and output";
    return r;
  }
  if (step.chained && step.scratch == nullptr) {
    r.diagnostic = "chained decode step needs a scratch buffer";
    return r;
  }
  for (std::size_t i = 0; i < n; ++i) {
    if (step.layers[i] == nullptr || !step.layers[i]->valid() || step.tables[i] == nullptr) {
      r.diagnostic = "decode step layer " + std::to_string(i) + " is not valid";
      return r;
    }
    if (step.layers[i]->config().geometry.hidden != step.layers[0]->config().geometry.hidden) {
      r.diagnostic = "decode step layers differ in hidden size";
      return r;
    }
  }
  const std::size_t rows = static_cast<std::size_t>(step.tokens) * step.layers[0]->config().geometry.hidden;
  for (std::size_t i = 0; i < n; ++i) {
    const float* x;
    float* y;
    if (step.chained) {
      // Ping-pong so the last layer writes y.
      const bool to_y = ((n - 1 - i) % 2) == 0;
      x = (i == 0) ? step.x : (to_y ? step.scratch : step.y);
      y = to_y ? step.y : step.scratch;
    } else {
      x = step.x + i * rows;
      y = step.y + i * rows;
    }
    auto d = step.layers[i]->decode_device(context, x, y, step.tokens, step.tables[i], step.chained);
    if (!d.executed) {
      r.diagnostic = "decode step layer " + std::to_string(i) + ": " + d.diagnostic;
      return r;
    }
  }
  r.executed = true;
  r.diagnostic = "decode step enqueued";
  return r;
}

HipGraph::~HipGraph() {
  if (exec_ != nullptr) {
    (void)osmd_set_device(device_);
    (void)osmd_graph_destroy(exec_);
  }
}

HipGraph::HipGraph(HipGraph&& o) noexcept : exec_(std::exchange(o.exec_, nullptr)), device_(o.device_) {}

HipGraph& HipGraph::operator=(HipGraph&& o) noexcept {
  if (this != &o) {
    if (exec_ != nullptr) {
      (void)osmd_set_device(device_);
      (void)osmd_graph_destroy(exec_);
    }
    exec_ = std::exchange(o.exec_, nullptr);
    device_ = o.device_;
  }
  return *this;
}

bool HipGraph::begin_capture(HipComputeContext& context, std::string* diagnostic) noexcept {
  if (!context.activate(diagnostic)) return false;
  const int rc = osmd_capture_begin(context.stream());
  if (rc != 0) return set_diag(diagnostic, hip_error("graph capture begin failed", rc)), false;
  return true;
}

std::optional<HipGraph> HipGraph::end_capture(HipComputeContext& context, std::string* diagnostic) noexcept {
  if (!context.activate(diagnostic)) return std::nullopt;
  osmd_graph exec = nullptr;
  const int rc = osmd_capture_end(context.stream(), &exec);
  if (rc != 0 || exec == nullptr)
    return set_diag(diagnostic, hip_error("graph capture end or instantiate failed", rc)), std::nullopt;
  HipGraph g;
  g.exec_ = exec;
  g.device_ = context.device();
  return g;
}

std::optional<HipGraph> HipGraph::capture_decode_step(HipComputeContext& context, const HipDecodeStep& step,
                                                      std::string* diagnostic) noexcept {
  try {
    // Reject what the step would reject before any capture begins.
    if (step.layers.empty() || step.tables.size() != step.layers.size() || step.x == nullptr ||
        step.y == nullptr || (step.chained && step.scratch == nullptr))
      return set_diag(diagnostic, "decode graph: invalid decode step"), std::nullopt;
    if (!begin_capture(context, diagnostic)) return std::nullopt;
    const HipDispatchResult enq = enqueue_decode_step(context, step);
    auto g = end_capture(context, diagnostic);  // always ends the capture
    if (!enq.executed) return set_diag(diagnostic, "decode graph: " + enq.diagnostic), std::nullopt;
    return g;
  } catch (const std::exception& e) {
    return set_diag(diagnostic, std::string("decode graph exception: ") + e.what()), std::nullopt;
  }
}

HipDispatchResult HipGraph::launch(HipComputeContext& context) noexcept {
  HipDispatchResult r;
  if (exec_ == nullptr) {
    r.diagnostic = "graph is not valid";
    return r;
  }
  if (!context.activate(&r.diagnostic)) return r;
  if (context.device() != device_) {
    r.diagnostic = "graph belongs to a different device";
    return r;
  }
  const int rc = osmd_graph_launch(exec_, context.stream());
  if (rc != 0) {
    r.diagnostic = hip_error("graph launch failed", rc);
    return r;
  }
  r.executed = true;
  r.diagnostic = "graph launched";
  return r;
}

}  // namespace osm
