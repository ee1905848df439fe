// Stream capture into one executable hipGraph (interface of cuda/graph.hpp in
// Enucatl/qw38). Capture never launches; launch() replays the executable.
#pragma once

#include "cuda/stream.hpp"

#include <hip/hip_runtime.h>

#include <utility>

namespace qw38::cuda {

class Graph {
 public:
  Graph() = default;
  Graph(Graph&& other) noexcept { swap(other); }
  Graph& operator=(Graph&& other) noexcept {
    if (this == &other) return *this;
    Graph old;
    old.swap(*this);
    swap(other);
    return *this;
  }
  ~Graph();
  Graph(Graph const&) = delete;
  Graph& operator=(Graph const&) = delete;
  static expected<Graph, Error> begin(Stream const&);
  expected<void, Error> finish();
  expected<void, Error> launch(Stream const&) const;
  bool empty() const noexcept { return exec_ == nullptr; }

 private:
  void swap(Graph& other) noexcept {
    std::swap(stream_, other.stream_);
    std::swap(device_, other.device_);
    std::swap(capturing_, other.capturing_);
    std::swap(graph_, other.graph_);
    std::swap(exec_, other.exec_);
  }
  hipStream_t stream_{};
  int device_{-1};
  bool capturing_{};
  hipGraph_t graph_{};
  hipGraphExec_t exec_{};
};

namespace testing {
void fail_next_graph_instantiation() noexcept;
}

// Public synchronous APIs reject a capturing stream before any launch.
expected<void, Error> require_uncaptured(Stream const&);

}  // namespace qw38::cuda
