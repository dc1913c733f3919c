// storage.cpp -- expert blobs read from a container directory with pread.
//
// PosixPreadExpertStorage (storage/posix_pread_expert_storage.cpp:98-187):
// layer L's experts sit back to back at a fixed stride in
// <dir>/packed_experts/layer_LL.bin (posix_pread_expert_storage.cpp:27-34);
// a read validates every request before any I/O, then reads the requests in
// parallel, and fails as a whole if any read fails or comes up short. The
// layer and expert counts and the stride are given by the caller (the
// reference takes them from the container's layout.json).
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <exception>
#include <limits>
#include <stdexcept>
#include <system_error>
#include <thread>

#include "osm_hip.hpp"

namespace osm {

namespace {

constexpr std::size_t kReadWorkers = 16;  // parallel preads per call at most

[[noreturn]] void throw_errno(const char* what, int error) {
  throw std::system_error(error, std::generic_category(), what);
}

}  // namespace

std::filesystem::path PosixPreadExpertStorage::layer_path(const std::filesystem::path& dir, std::uint32_t layer) {
  char name[32];
  std::snprintf(name, sizeof(name), "layer_%02u.bin", layer);
  return dir / "packed_experts" / name;
}

PosixPreadExpertStorage::PosixPreadExpertStorage(std::filesystem::path container_dir, std::uint32_t layers,
                                                 std::uint32_t experts, std::size_t stride)
    : dir_(std::move(container_dir)), layers_(layers), experts_(experts), stride_(stride),
      fds_(layers, -1) {
  if (layers == 0 || experts == 0 || stride == 0)
    throw std::invalid_argument("posix expert storage: layers, experts and stride must be non-zero");
  if (stride > static_cast<std::size_t>(std::numeric_limits<ssize_t>::max()))
    throw std::invalid_argument("posix expert storage: expert stride exceeds pread size range");
}

PosixPreadExpertStorage::~PosixPreadExpertStorage() {
  for (const int fd : fds_)
    if (fd >= 0) ::close(fd);
}

int PosixPreadExpertStorage::fd_for_layer(std::uint32_t layer) {
  std::scoped_lock lock(mutex_);
  if (fds_[layer] >= 0) return fds_[layer];
  const auto path = layer_path(dir_, layer);
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) throw_errno("open expert layer", errno);
  fds_[layer] = fd;
  return fd;
}

void PosixPreadExpertStorage::read_experts(std::span<ExpertReadRequest> requests) {
  if (requests.empty()) return;
  struct Prepared {
    int fd;
    off_t offset;
    std::byte* destination;
  };
  // Everything is resolved before the first read, so a bad request fails
  // the call without partial I/O (posix_pread_expert_storage.cpp:118-152).
  std::vector<Prepared> prepared;
  prepared.reserve(requests.size());
  for (auto& r : requests) {
    if (r.id.layer >= layers_) throw std::out_of_range("posix expert storage: layer index out of range");
    if (r.id.expert >= experts_) throw std::out_of_range("posix expert storage: expert index out of range");
    if (r.destination.size() < stride_)
      throw std::invalid_argument("posix expert storage: destination smaller than expert stride");
    const std::uint64_t offset = static_cast<std::uint64_t>(r.id.expert) * stride_;
    if (offset > static_cast<std::uint64_t>(std::numeric_limits<off_t>::max()))
      throw std::runtime_error("posix expert storage: expert offset exceeds off_t range");
    prepared.push_back({fd_for_layer(r.id.layer), static_cast<off_t>(offset), r.destination.data()});
  }
  // One pread per request, spread over at most kReadWorkers threads; a read
  // that returns less than asked continues where it stopped, and end of
  // file before the stride is a short read.
  std::vector<std::exception_ptr> failures(prepared.size());
  auto read_one = [&](std::size_t i) {
    try {
      const Prepared& p = prepared[i];
      std::size_t done = 0;
      while (done < stride_) {
        const ssize_t got = ::pread(p.fd, p.destination + done, stride_ - done, p.offset + static_cast<off_t>(done));
        if (got < 0) {
          if (errno == EINTR) continue;
          throw_errno("pread expert", errno);
        }
        if (got == 0) throw std::runtime_error("posix expert storage: short expert read");
        done += static_cast<std::size_t>(got);
      }
    } catch (...) {
      failures[i] = std::current_exception();
    }
  };
  const std::size_t workers = std::min(prepared.size(), kReadWorkers);
  if (workers <= 1) {
    for (std::size_t i = 0; i < prepared.size(); ++i) read_one(i);
  } else {
    std::vector<std::jthread> pool;
    pool.reserve(workers);
    for (std::size_t w = 0; w < workers; ++w)
      pool.emplace_back([&, w] {
        for (std::size_t i = w; i < prepared.size(); i += workers) read_one(i);
      });
    pool.clear();  // joins: every worker's writes are complete
  }
  for (const auto& f : failures)
    if (f) std::rethrow_exception(f);
}

}  // namespace osm
