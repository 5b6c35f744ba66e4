// pet/graph.hpp -- record-and-replay of a sequence of the path's calls as one
// HIP graph launch, the role of the reference's GraphCache
// (peterspackman/pet-kokkos include/pet/graph.hpp) for a C++ caller.
//
// run(key, work) runs work() eagerly the first time it sees key, captures it
// (hipStreamBeginCapture on `stream`, relaxed mode) the second time, and from
// then on launches the instantiated graph: the same kernels in the same order
// on the same buffers, so the results are bit-identical to an eager run. The
// key must name everything the recorded work depends on (shapes, the buffers
// it reads and writes, the workspace's allocations), since a replay reuses the
// recorded pointers. The least recently used graph is dropped past kKeep. A
// capture that fails (an allocation or a host synchronisation inside work)
// clears the sticky error and switches the cache to eager work for good.
//
// Everything this library enqueues can be captured: it clears with kernels,
// never hipMemsetAsync, and a warm pet::Workspace allocates nothing.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <vector>

namespace pet {

class GraphCache {
 public:
  using Key = std::vector<std::uintptr_t>;
  static constexpr std::size_t kKeep = 8;

  explicit GraphCache(hipStream_t stream = nullptr) : stream_(stream) {}
  GraphCache(const GraphCache&) = delete;
  GraphCache& operator=(const GraphCache&) = delete;
  ~GraphCache() { clear(); }

  bool broken() const { return broken_; }
  std::size_t size() const { return graphs_.size(); }

  template <class F>
  void run(const Key& key, F&& work) {
    if (broken_) return work();
    ++tick_;
    for (Entry& e : graphs_)
      if (e.key == key) {
        e.used = tick_;
        if (hipGraphLaunch(e.exec, stream_) != hipSuccess) throw_error();
        return;
      }
    if (std::find(seen_.begin(), seen_.end(), key) == seen_.end()) {
      seen_.push_back(key);
      if (seen_.size() > 2 * kKeep) seen_.erase(seen_.begin());
      return work();  // first sight: eagerly
    }
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool ok = hipStreamBeginCapture(stream_, hipStreamCaptureModeRelaxed) == hipSuccess;
    if (ok) {
      work();
      ok = hipStreamEndCapture(stream_, &graph) == hipSuccess && graph &&
           hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
    }
    if (graph) (void) hipGraphDestroy(graph);
    if (!ok) {
      (void) hipGetLastError();
      broken_ = true;
      return work();
    }
    if (graphs_.size() >= kKeep) {
      auto lru = std::min_element(graphs_.begin(), graphs_.end(),
                                  [](const Entry& a, const Entry& b) { return a.used < b.used; });
      (void) hipGraphExecDestroy(lru->exec);
      graphs_.erase(lru);
    }
    graphs_.push_back({key, exec, tick_});
    if (hipGraphLaunch(exec, stream_) != hipSuccess) throw_error();  // the capture did not run the work
  }

  void clear() {
    for (Entry& e : graphs_) (void) hipGraphExecDestroy(e.exec);
    graphs_.clear();
    seen_.clear();
  }

 private:
  struct Entry {
    Key key;
    hipGraphExec_t exec;
    std::uint64_t used;
  };
  [[noreturn]] static void throw_error() { throw std::runtime_error("pet: graph launch failed"); }
  hipStream_t stream_;
  std::vector<Entry> graphs_;
  std::vector<Key> seen_;
  std::uint64_t tick_ = 0;
  bool broken_ = false;
};

}  // namespace pet
