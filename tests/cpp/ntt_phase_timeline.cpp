// Phase timeline of the single-pass forward NTT (ntt_fwd_1p) at config 2:
// one forward NTT of 2 polys x 32 limbs, N = 2^16, 30-bit primes. Needs the
// instrumented library (cheddar-fhe_amd/build.py --phase-timestamps DIR),
// whose waves record the 100 MHz real-time clock at each phase boundary;
// prints, per boundary, the spread over all waves of the time since the
// first wave started. The argument (default 500) is the number of forwards
// run back to back, first without and then with timestamps, so the table
// (the last forward's) shows the kernel at sustained clocks. Exits with an
// error on the product library, which has no timestamp hook.
#include <hip/hip_runtime.h>
#include <dlfcn.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "cheddar_amd.h"

#define CK(x)                                                         \
  do {                                                                \
    hipError_t e_ = (x);                                              \
    if (e_ != hipSuccess) {                                           \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), \
                  __LINE__);                                          \
      std::exit(1);                                                   \
    }                                                                 \
  } while (0)

namespace {

bool is_prime(uint64_t n) {
  for (uint64_t d = 2; d * d <= n; d++)
    if (n % d == 0) return false;
  return n >= 2;
}

// the count largest primes below 2^bits that are 1 mod 2^17, descending (the
// benchmark's chain for config 2)
std::vector<uint32_t> ntt_primes(int bits, int count) {
  std::vector<uint32_t> r;
  const uint64_t step = uint64_t{1} << 17;
  uint64_t q = ((uint64_t{1} << bits) - 1) / step * step + 1;
  while ((int)r.size() < count) {
    if (is_prime(q)) r.push_back((uint32_t)q);
    q -= step;
  }
  return r;
}

}  // namespace

int main(int argc, char **argv) {
  const int warmup = argc > 1 ? std::max(1, std::atoi(argv[1])) : 500;
  using set_fn = int (*)(unsigned long long *, int);
  auto set_ts = reinterpret_cast<set_fn>(
      dlsym(RTLD_DEFAULT, "chd_debug_phase_timestamps"));
  if (set_ts == nullptr) {
    std::printf("the loaded libcheddar_amd.so is not the instrumented build "
                "(build.py --phase-timestamps)\n");
    return 1;
  }
  const int N = 1 << 16, L = 32, P = 2;
  // ntt_fwd_1p: 4 workgroups of 16 waves per limb
  const int waves = 4 * L * P * 16;
  std::vector<uint32_t> pr = ntt_primes(30, L);
  chd_ntt_plan *plan = nullptr;
  if (chd_ntt_plan_create(&plan, 16, pr.data(), L)) {
    std::printf("%s\n", chd_last_error());
    return 1;
  }
  const size_t words = (size_t)P * L * N;
  std::vector<uint32_t> h(words);
  for (size_t i = 0; i < words; i++)
    h[i] = (uint32_t)((i * 2654435761u) % pr[(i / N) % L]);
  uint32_t *src, *dst;
  unsigned long long *ts;
  CK(hipMalloc(&src, words * 4));
  CK(hipMalloc(&dst, words * 4));
  CK(hipMalloc(&ts, (size_t)waves * 8 * sizeof(unsigned long long)));
  CK(hipMemcpy(src, h.data(), words * 4, hipMemcpyHostToDevice));
  std::vector<unsigned long long> t((size_t)waves * 8);
  const char *names[7] = {"start",          "round-1 loads",
                          "round 1",        "barrier passed",
                          "round 2",        "round 3",
                          "round 4+stores"};
  // warm-up: forwards back to back without timestamps (sustained clocks)
  if (set_ts(nullptr, 0)) {
    std::printf("%s\n", chd_last_error());
    return 1;
  }
  for (int rep = 0; rep < warmup; rep++)
    if (chd_ntt_forward(plan, dst, src, L, P, 0, nullptr)) {
      std::printf("%s\n", chd_last_error());
      return 1;
    }
  // the instrumented forward, right behind the warm-up ones on the stream
  CK(hipMemsetAsync(ts, 0, (size_t)waves * 8 * sizeof(unsigned long long),
                    nullptr));
  CK(hipDeviceSynchronize());
  if (set_ts(ts, waves)) {
    std::printf("%s\n", chd_last_error());
    return 1;
  }
  for (int rep = 0; rep < warmup; rep++)
    if (chd_ntt_forward(plan, dst, src, L, P, 0, nullptr)) {
      std::printf("%s\n", chd_last_error());
      return 1;
    }
  CK(hipDeviceSynchronize());
  CK(hipMemcpy(t.data(), ts, t.size() * sizeof(unsigned long long),
               hipMemcpyDeviceToHost));
  // every forward above wrote the same slots: the table is the last one
  unsigned long long t0 = ~0ull, tend = 0;
  for (int w = 0; w < waves; w++) {
    t0 = std::min(t0, t[w * 8]);
    tend = std::max(tend, t[w * 8 + 6]);
  }
  std::printf("last of %d instrumented forwards (after %d plain ones): "
              "first wave start -> last wave end %.2f us\n",
              warmup, warmup, (tend - t0) / 100.0);
  for (int k = 0; k < 7; k++) {
    std::vector<double> v;
    for (int w = 0; w < waves; w++)
      if (t[w * 8 + k]) v.push_back((t[w * 8 + k] - t0) / 100.0);
    if (v.empty()) continue;
    std::sort(v.begin(), v.end());
    std::printf("%-15s waves %4zu  min %6.2f  p10 %6.2f  p50 %6.2f  "
                "p90 %6.2f  max %6.2f us\n",
                names[k], v.size(), v[0], v[v.size() / 10], v[v.size() / 2],
                v[v.size() * 9 / 10], v.back());
  }
  set_ts(nullptr, 0);
  CK(hipFree(ts));
  CK(hipFree(dst));
  CK(hipFree(src));
  chd_ntt_plan_destroy(plan);
  return 0;
}
