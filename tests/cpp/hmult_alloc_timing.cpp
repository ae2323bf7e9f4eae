// Host enqueue and GPU time of Context::HMult at config 4 (N = 2^16, L = 24,
// alpha = 8, dnum 3, merged rescale) when the caller makes a new result
// ciphertext per call, as the reference's callers do (Context.cpp:862-871
// writes into a caller-made Ciphertext), against a result allocated once:
//   preallocated  the result's memory is reused, no allocation per call
//   pool          a new Ciphertext per call, memory from the device pool
//   hipMalloc     per call hipMalloc + hipFree of the result (what a
//                 DeviceVector without a pool does)
// Prints one line per variant: mean host microseconds per call to enqueue
// (the loop without any wait) and GPU microseconds per call (events around
// the loop). Needs a HIP device.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>
#include <cstdio>
#include <vector>

#include "cheddar.h"

using namespace cheddar;
using word = uint32_t;
using Ct = Ciphertext<word>;

namespace {
constexpr int kLogN = 16;
constexpr size_t kN = size_t{1} << kLogN;

std::vector<word> primes(int bits, int count) {
  std::vector<word> r;
  const uint64_t step = 1u << 17;
  uint64_t q = ((uint64_t{1} << bits) - 1) / step * step + 1;
  auto is_prime = [](uint64_t n) {
    for (uint64_t d = 2; d * d <= n; d++)
      if (n % d == 0) return false;
    return true;
  };
  while (static_cast<int>(r.size()) < count) {
    if (is_prime(q)) r.push_back(static_cast<word>(q));
    q -= step;
  }
  return r;
}

void fill(word *p, size_t words, word q) {  // any residues below q
  std::vector<word> h(words);
  for (size_t i = 0; i < words; i++) h[i] = static_cast<word>(i * 2654435761u) % q;
  HipCheck(hipMemcpy(p, h.data(), words * sizeof(word), hipMemcpyHostToDevice),
           "hipMemcpy");
}

template <typename F>
void timed(const char *name, int iters, F body) {
  for (int i = 0; i < 3; i++) body();
  HipCheck(hipDeviceSynchronize(), "hipDeviceSynchronize");
  hipEvent_t e0, e1;
  HipCheck(hipEventCreate(&e0), "hipEventCreate");
  HipCheck(hipEventCreate(&e1), "hipEventCreate");
  HipCheck(hipEventRecord(e0, nullptr), "hipEventRecord");
  const auto t0 = std::chrono::steady_clock::now();
  for (int i = 0; i < iters; i++) body();
  const auto t1 = std::chrono::steady_clock::now();
  HipCheck(hipEventRecord(e1, nullptr), "hipEventRecord");
  HipCheck(hipEventSynchronize(e1), "hipEventSynchronize");
  float ms = 0;
  HipCheck(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
  const double host_us =
      std::chrono::duration<double, std::micro>(t1 - t0).count() / iters;
  std::printf("%-14s host_enqueue_us_per_call %8.2f  gpu_us_per_call %8.2f\n",
              name, host_us, 1e3 * ms / iters);
  std::fflush(stdout);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
}
}  // namespace

int main(int argc, char **argv) {
  const int iters = argc > 1 ? std::atoi(argv[1]) : 200;
  const int L = 24, alpha = 8;
  const std::vector<word> main_p = primes(30, L), aux_p = primes(31, alpha);
  std::vector<std::pair<int, int>> levels;
  for (int i = 1; i <= L; i++) levels.emplace_back(i, 0);
  Parameter<word> param(kLogN, 0x1p30, L - 1, levels, main_p, aux_p);
  auto ctx = Context<word>::Create(param);
  const NPInfo np = param.LevelToNP(L - 1);
  Ct a(np), b(np);
  for (Ct *c : {&a, &b}) {
    fill(c->bx_.data(), c->bx_.size(), main_p.back());
    fill(c->ax_.data(), c->ax_.size(), main_p.back());
    c->SetScale(0x1p30);
  }
  EvaluationKey<word> key(param.LevelToNP(param.max_level_, alpha),
                          param.dnum_);
  for (int g = 0; g < param.dnum_; g++) {
    fill(key.bx_[g].data(), key.bx_[g].size(), main_p.back());
    fill(key.ax_[g].data(), key.ax_[g].size(), main_p.back());
  }
  const size_t out_words = static_cast<size_t>(L - 1) * kN;
  const auto ref = Context<word>::RefOfKey(key);

  Ct pre;
  timed("preallocated", iters, [&] { ctx->HMult(pre, a, b, key, true); });
  timed("pool", iters, [&] {
    Ct res;
    ctx->HMult(res, a, b, key, true);
  });
  timed("hipMalloc", iters, [&] {
    word *rb = nullptr, *ra = nullptr;
    HipCheck(hipMalloc(&rb, out_words * sizeof(word)), "hipMalloc");
    HipCheck(hipMalloc(&ra, out_words * sizeof(word)), "hipMalloc");
    ctx->HMultV(L - 1, {rb, ra, nullptr}, {a.bx_.data(), a.ax_.data(), nullptr},
                {b.bx_.data(), b.ax_.data(), nullptr}, ref, true);
    HipCheck(hipFree(rb), "hipFree");
    HipCheck(hipFree(ra), "hipFree");
  });
  const MemoryPool::Stats st = MemoryPool::Current().GetStats();
  std::printf("pool device_allocations %zu reuses %zu\n",
              st.device_allocations, st.reuses);
  return 0;
}
