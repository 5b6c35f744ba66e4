// pet/replay.hpp -- a caller's repeated device work kept as instantiated HIP
// graphs and launched with one call (the role the reference gives its graph
// cache, include/pet/graph.hpp of peterspackman/pet-kokkos; the design here is
// this library's own).
//
// A caller names a unit of work by a Signature: a list of words (shapes, flags
// and the device addresses the work reads and writes) folded into a 64-bit
// digest. StepRecorder::launch(sig, work) then
//   - runs work() eagerly for the signature's first `warm_runs` calls, so
//     every lazily grown buffer reaches its final address before anything is
//     recorded;
//   - on the next call records work() by stream capture (global mode off:
//     relaxed), instantiates it, and launches the instance;
//   - from then on launches the instance only: the same kernels in the same
//     order on the same addresses, so the results are bit-identical to an
//     eager run.
// Live instances are held in recency order; past `max_live` the least
// recently launched is destroyed. A signature whose capture fails (work that
// allocates or synchronises the host) is marked eager-only, the sticky error
// is cleared and a dangling capture ended; other signatures keep recording.
// Counters (launches, records, refusals, evictions) let a caller or a test see
// what happened.
//
// Everything this library enqueues can be captured: it clears with kernels,
// never hipMemsetAsync, and a warm pet::Workspace allocates nothing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <initializer_list>
#include <iterator>
#include <list>
#include <stdexcept>
#include <unordered_map>
#include <vector>

namespace pet {

// The words that identify a unit of recorded work, with their digest.
class Signature {
 public:
  Signature() = default;
  Signature(std::initializer_list<std::uint64_t> words) {
    for (std::uint64_t w : words) add(w);
  }
  Signature& add(std::uint64_t w) {
    words_.push_back(w);
    // splitmix64 finaliser over the running digest and the new word
    std::uint64_t z = digest_ + 0x9e3779b97f4a7c15ull + w;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    digest_ = z ^ (z >> 31);
    return *this;
  }
  template <class T>
  Signature& add(const T* p) {
    return add(std::uint64_t(reinterpret_cast<std::uintptr_t>(p)));
  }
  std::uint64_t digest() const { return digest_; }
  bool operator==(const Signature& o) const { return digest_ == o.digest_ && words_ == o.words_; }

 private:
  std::vector<std::uint64_t> words_;
  std::uint64_t digest_ = 0x6a09e667f3bcc908ull;
};

struct SignatureDigest {
  std::size_t operator()(const Signature& s) const { return std::size_t(s.digest()); }
};

class StepRecorder {
 public:
  struct Counters {
    std::uint64_t eager = 0;      // calls run eagerly (warming or eager-only)
    std::uint64_t records = 0;    // captures instantiated
    std::uint64_t launches = 0;   // instance launches (a record's first included)
    std::uint64_t refusals = 0;   // captures that failed (signature now eager-only)
    std::uint64_t evictions = 0;  // instances destroyed to stay within max_live
  };

  explicit StepRecorder(hipStream_t stream, int warm_runs = 1, std::size_t max_live = 8)
      : stream_(stream), warm_runs_(warm_runs < 0 ? 0 : warm_runs), max_live_(max_live ? max_live : 1) {}
  StepRecorder(const StepRecorder&) = delete;
  StepRecorder& operator=(const StepRecorder&) = delete;
  ~StepRecorder() { forget(); }

  const Counters& counters() const { return n_; }
  std::size_t live() const { return recent_.size(); }

  template <class Work>
  void launch(const Signature& sig, Work&& work) {
    if (plans_.size() >= 4 * max_live_ && !plans_.count(sig)) drop_cold();
    Plan& p = plans_[sig];
    if (p.state == Plan::kLive) {
      recent_.splice(recent_.begin(), recent_, p.pos);  // most recent first
      return go(p.exec);
    }
    if (p.state == Plan::kEagerOnly || p.eager_runs < warm_runs_) {
      ++p.eager_runs, ++n_.eager;
      return work();
    }
    hipGraphExec_t exec = record(work);
    if (!exec) {
      p.state = Plan::kEagerOnly;
      ++n_.refusals, ++n_.eager;
      return work();  // the failed capture ran nothing
    }
    ++n_.records;
    p.state = Plan::kLive, p.exec = exec;
    recent_.push_front(sig);
    p.pos = recent_.begin();
    while (recent_.size() > max_live_) retire(recent_.back());
    go(exec);  // a capture records the work without running it
  }

  // Destroys every instance and forgets every signature (e.g. when the buffers
  // the signatures name are freed or regrown).
  void forget() {
    for (auto& kv : plans_)
      if (kv.second.state == Plan::kLive) (void) hipGraphExecDestroy(kv.second.exec);
    plans_.clear();
    recent_.clear();
  }

 private:
  struct Plan {
    enum State { kWarming, kLive, kEagerOnly } state = kWarming;
    int eager_runs = 0;
    hipGraphExec_t exec = nullptr;
    std::list<Signature>::iterator pos;
  };

  template <class Work>
  hipGraphExec_t record(Work& work) {
    if (hipStreamBeginCapture(stream_, hipStreamCaptureModeRelaxed) != hipSuccess) {
      (void) hipGetLastError();
      return nullptr;
    }
    bool threw = false;
    try {
      work();
    } catch (...) {
      threw = true;
    }
    hipGraph_t g = nullptr;
    const bool ended = hipStreamEndCapture(stream_, &g) == hipSuccess && g;
    hipGraphExec_t exec = nullptr;
    if (ended && !threw && hipGraphInstantiate(&exec, g, nullptr, nullptr, 0) != hipSuccess) exec = nullptr;
    if (g) (void) hipGraphDestroy(g);
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream_, &status) == hipSuccess && status != hipStreamCaptureStatusNone) {
      hipGraph_t dangling = nullptr;
      (void) hipStreamEndCapture(stream_, &dangling);
      if (dangling) (void) hipGraphDestroy(dangling);
    }
    if (!exec) (void) hipGetLastError();
    return exec;
  }

  // Signatures not holding an instance (warming or eager-only) are forgotten,
  // so that a caller cycling through many keys keeps the table bounded.
  void drop_cold() {
    for (auto it = plans_.begin(); it != plans_.end();)
      it = it->second.state == Plan::kLive ? std::next(it) : plans_.erase(it);
  }

  void go(hipGraphExec_t exec) {
    ++n_.launches;
    if (hipGraphLaunch(exec, stream_) != hipSuccess) throw std::runtime_error("pet: graph launch failed");
  }

  void retire(const Signature& sig) {
    auto it = plans_.find(sig);
    if (it == plans_.end()) return;
    (void) hipGraphExecDestroy(it->second.exec);
    recent_.erase(it->second.pos);
    plans_.erase(it);  // a retired signature warms up again if it returns
    ++n_.evictions;
  }

  hipStream_t stream_;
  int warm_runs_;
  std::size_t max_live_;
  std::unordered_map<Signature, Plan, SignatureDigest> plans_;
  std::list<Signature> recent_;
  Counters n_;
};

}  // namespace pet
