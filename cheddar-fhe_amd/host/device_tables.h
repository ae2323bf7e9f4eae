// Device memory RAII and the per-prime-chain constant tables the kernels
// read (twiddles, primes, Montgomery and fp64 constants).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "cheddar_kernels.h"

namespace cheddar {

// Throws with the HIP error text; C-ABI entry points catch and convert.
void HipCheck(hipError_t e, const char *what);

// Owning device allocation (hipMalloc). Move-only.
class DevBuf {
 public:
  DevBuf() = default;
  explicit DevBuf(size_t bytes) { Resize(bytes); }
  ~DevBuf() { Release(); }
  DevBuf(const DevBuf &) = delete;
  DevBuf &operator=(const DevBuf &) = delete;
  DevBuf(DevBuf &&o) noexcept : ptr_(o.ptr_), bytes_(o.bytes_) {
    o.ptr_ = nullptr;
    o.bytes_ = 0;
  }
  DevBuf &operator=(DevBuf &&o) noexcept {
    if (this != &o) {
      Release();
      ptr_ = o.ptr_;
      bytes_ = o.bytes_;
      o.ptr_ = nullptr;
      o.bytes_ = 0;
    }
    return *this;
  }
  void Resize(size_t bytes);
  void Upload(const void *host, size_t bytes);
  template <typename T>
  void Upload(const std::vector<T> &v) {
    Resize(v.size() * sizeof(T));
    Upload(v.data(), v.size() * sizeof(T));
  }
  template <typename T>
  T *as() const {
    return static_cast<T *>(ptr_);
  }
  size_t bytes() const { return bytes_; }

 private:
  void Release();
  void *ptr_ = nullptr;
  size_t bytes_ = 0;
};

// Tables for a chain of primes in chain order (each prime q = 1 mod 2N).
class ChainTables {
 public:
  ChainTables(int log_degree, const std::vector<uint32_t> &primes);
  const chd_tables &tables() const { return tab_; }
  int size() const { return static_cast<int>(primes_.size()); }
  const std::vector<uint32_t> &primes() const { return primes_; }
  // per-prime reference-form constants (src/core/NTT.cu:1255-1265)
  const uint32_t *inv_degree() const { return ninv_.as<uint32_t>(); }
  const uint32_t *inv_degree_mont() const { return ninv_mont_.as<uint32_t>(); }
  const uint32_t *mont_converter() const { return r2_.as<uint32_t>(); }

 private:
  std::vector<uint32_t> primes_;
  DevBuf q_, qinv_, tw_, itw_, twist_;
  DevBuf ninv_, ninv_mont_, r2_;
  chd_tables tab_{};
};

}  // namespace cheddar
