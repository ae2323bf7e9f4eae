// Device memory pool behind DeviceVector: the reference's MemoryPool
// (src/core/MemoryPool.cpp:5-35, include/core/MemoryPool.h), an RMM
// binning resource over the stream-ordered CUDA pool, rebuilt on HIP.
//
// One pool per GPU, created on first use and kept until the process ends
// (like RMM's per-device resource). Allocation sizes are rounded up to the
// reference's bins (MemoryPool.cpp:10-31): x4 steps from 512 B below one
// limb, x2 steps from one limb below alpha limbs, alpha-limb steps up to
// (L + alpha) limbs. Each bin keeps the blocks released to it with the
// stream they were released on and an event recorded there: a request on
// the same stream takes such a block at once (stream order makes it safe),
// a request on another stream first makes its stream wait for that event.
// New blocks come from hipMalloc when a bin is empty; requests beyond the
// largest bin go to HIP's stream-ordered allocator (hipMallocAsync /
// hipFreeAsync on the request's stream), as the reference's do to its
// upstream resource.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <mutex>
#include <set>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace cheddar {

class MemoryPool {
 public:
  // the pool of the current device
  static MemoryPool &Current();

  // the reference's bins for a parameter set (limb = degree words); bins
  // of several parameter sets add up
  void AddBins(size_t limb_bytes, int alpha, int L);
  // a block of at least `bytes` usable in stream order on `stream`;
  // *reserved is the size actually held (the bin size), to be passed back
  void *Allocate(size_t bytes, hipStream_t stream, size_t *reserved);
  void Deallocate(void *p, size_t reserved, hipStream_t stream) noexcept;
  // returns every cached block to the driver once its release event has
  // completed; returns the bytes freed
  size_t ReleaseCached();

  struct Stats {
    size_t device_allocations = 0;  // hipMalloc calls for bin blocks
    size_t reuses = 0;              // requests served from a free list
    size_t cached_bytes = 0;        // bytes in free lists
    size_t upstream_allocations = 0;  // requests beyond the largest bin
  };
  Stats GetStats();
  std::vector<size_t> Bins();

 private:
  MemoryPool() = default;
  struct Block {
    void *p;
    hipStream_t stream;
    hipEvent_t released;  // nullptr: the release was synchronised
  };
  hipEvent_t TakeEvent();
  size_t ReleaseCachedLocked();
  std::mutex mu_;
  std::set<size_t> bins_;
  std::unordered_map<size_t, std::vector<Block>> free_;
  std::unordered_set<void *> upstream_;
  std::vector<hipEvent_t> spare_events_;
  Stats stats_;
};

}  // namespace cheddar
