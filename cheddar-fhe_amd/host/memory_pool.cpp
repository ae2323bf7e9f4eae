#include "memory_pool.h"

#include <stdexcept>
#include <string>

#include "device_tables.h"

namespace cheddar {

MemoryPool &MemoryPool::Current() {
  static std::mutex mu;
  // never destroyed: blocks may be released by objects that outlive any
  // static destructor order, and the driver reclaims memory at exit
  static std::vector<MemoryPool *> *pools = new std::vector<MemoryPool *>();
  int dev = 0;
  HipCheck(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= static_cast<int>(pools->size())) pools->resize(dev + 1, nullptr);
  if ((*pools)[dev] == nullptr) (*pools)[dev] = new MemoryPool();
  return *(*pools)[dev];
}

// MemoryPool.cpp:10-31
void MemoryPool::AddBins(size_t limb_bytes, int alpha, int L) {
  if (limb_bytes == 0 || alpha < 1 || L < 1)
    throw std::invalid_argument("MemoryPool: invalid parameters");
  std::lock_guard<std::mutex> lock(mu_);
  size_t bin = 512;
  for (; bin < limb_bytes; bin *= 4) bins_.insert(bin);
  bin = limb_bytes;
  const size_t chunk = static_cast<size_t>(alpha) * limb_bytes;
  for (; bin < chunk; bin *= 2) bins_.insert(bin);
  bin = chunk;
  const size_t max_size = static_cast<size_t>(L + alpha) * limb_bytes;
  for (; bin < max_size; bin += chunk) bins_.insert(bin);
  bins_.insert(max_size);
}

hipEvent_t MemoryPool::TakeEvent() {
  if (!spare_events_.empty()) {
    hipEvent_t e = spare_events_.back();
    spare_events_.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess)
    return nullptr;
  return e;
}

void *MemoryPool::Allocate(size_t bytes, hipStream_t stream,
                           size_t *reserved) {
  *reserved = 0;
  if (bytes == 0) return nullptr;
  std::lock_guard<std::mutex> lock(mu_);
  const auto bin = bins_.lower_bound(bytes);
  void *p = nullptr;
  if (bin == bins_.end()) {
    HipCheck(hipMallocAsync(&p, bytes, stream), "hipMallocAsync");
    upstream_.insert(p);
    stats_.upstream_allocations++;
    *reserved = bytes;
    return p;
  }
  const size_t size = *bin;
  std::vector<Block> &list = free_[size];
  if (!list.empty()) {
    // newest first: a block released on this stream needs no wait
    size_t pick = list.size() - 1;
    for (size_t i = list.size(); i-- > 0;)
      if (list[i].stream == stream) {
        pick = i;
        break;
      }
    const Block b = list[pick];
    if (b.stream != stream && b.released != nullptr)
      HipCheck(hipStreamWaitEvent(stream, b.released, 0),
               "hipStreamWaitEvent");
    list.erase(list.begin() + static_cast<std::ptrdiff_t>(pick));
    if (b.released != nullptr) spare_events_.push_back(b.released);
    stats_.reuses++;
    stats_.cached_bytes -= size;
    *reserved = size;
    return b.p;
  }
  if (hipMalloc(&p, size) != hipSuccess) {
    // out of device memory: give the cached blocks back and try once more
    (void)hipGetLastError();
    ReleaseCachedLocked();
    HipCheck(hipMalloc(&p, size), "hipMalloc");
  }
  stats_.device_allocations++;
  *reserved = size;
  return p;
}

void MemoryPool::Deallocate(void *p, size_t reserved,
                            hipStream_t stream) noexcept {
  if (p == nullptr) return;
  std::lock_guard<std::mutex> lock(mu_);
  if (upstream_.erase(p) != 0) {
    (void)hipFreeAsync(p, stream);
    return;
  }
  hipEvent_t e = TakeEvent();
  if (e != nullptr && hipEventRecord(e, stream) != hipSuccess) {
    (void)hipEventDestroy(e);
    e = nullptr;
  }
  if (e == nullptr) (void)hipStreamSynchronize(stream);
  try {
    free_[reserved].push_back(Block{p, stream, e});
    stats_.cached_bytes += reserved;
  } catch (...) {
    // no room to cache it: give it back once its stream is done with it
    // (nothing here may throw: this function is noexcept)
    if (e != nullptr) {
      (void)hipEventSynchronize(e);
      (void)hipEventDestroy(e);
    }
    (void)hipFree(p);
  }
}

size_t MemoryPool::ReleaseCached() {
  std::lock_guard<std::mutex> lock(mu_);
  return ReleaseCachedLocked();
}

size_t MemoryPool::ReleaseCachedLocked() {
  size_t freed = 0;
  for (auto &[size, list] : free_) {
    for (const Block &b : list) {
      if (b.released != nullptr) {
        (void)hipEventSynchronize(b.released);
        spare_events_.push_back(b.released);
      }
      (void)hipFree(b.p);
      freed += size;
    }
    list.clear();
  }
  stats_.cached_bytes = 0;
  return freed;
}

MemoryPool::Stats MemoryPool::GetStats() {
  std::lock_guard<std::mutex> lock(mu_);
  return stats_;
}

std::vector<size_t> MemoryPool::Bins() {
  std::lock_guard<std::mutex> lock(mu_);
  return std::vector<size_t>(bins_.begin(), bins_.end());
}

}  // namespace cheddar
