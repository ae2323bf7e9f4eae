// Constant-table dump built against the reference's own host-only headers.
//
// TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile (target `ref`) from
// this file plus the reference headers where they lie
// (/root/reference/include/common/PrimeUtils.h, CommonUtils.h), output into
// oracle/_ref/. It pins the oracle's number-theory constants (smallest
// generator, psi, q^-1 mod 2^32, Montgomery twiddles, ModSwitch tables) to
// the reference's implementation of the same primitives.
//
// Usage: refcheck <log_n> <num_src> <num_dst> <prime>...   (src then dst)
// Prints, per prime: q g psi qinv N^-1 ToMont(N^-1) R^2 and the first and a
// sampled set of twiddles; then the ModSwitch tables for src -> dst
// (ModSwitch.cu:320-370 loop structure, driven by primeutil:: primitives).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "common/CommonUtils.h"
#include "common/PrimeUtils.h"

using namespace cheddar;
using word = uint32_t;

int main(int argc, char **argv) {
  if (argc < 4) return 2;
  int log_n = std::atoi(argv[1]);
  int ns = std::atoi(argv[2]);
  int nd = std::atoi(argv[3]);
  std::vector<word> primes;
  for (int i = 4; i < argc; i++)
    primes.push_back(static_cast<word>(std::strtoul(argv[i], nullptr, 10)));
  if (static_cast<int>(primes.size()) != ns + nd) return 2;
  int n = 1 << log_n;

  // NTT.cu:1233-1299 table recipe, through the reference's primitives.
  for (word p : primes) {
    word g = primeutil::FindGenerator(p);
    word psi = primeutil::FindPrimitiveMthRoot(2 * n, p);
    word psi_inv = primeutil::InvMod<word>(psi, p);
    int32_t qinv = primeutil::InvModBase<word>(p);
    word ninv = primeutil::InvMod<word>(n, p);
    word ninv_m = primeutil::ToMontgomery<word>(ninv, p);
    word r2 = primeutil::ToMontgomery(primeutil::ToMontgomery<word>(1, p), p);
    std::vector<word> pr(n), pir(n);
    pr[0] = 1;
    pir[0] = 1;
    for (int j = 1; j < n; j++) {
      pr[j] = primeutil::MultMod(pr[j - 1], psi, p);
      pir[j] = primeutil::MultMod(pir[j - 1], psi_inv, p);
    }
    BitReverseVector(pr);
    BitReverseVector(pir);
    std::printf("prime %u %u %u %d %u %u %u\n", p, g, psi, qinv, ninv, ninv_m,
                r2);
    std::printf("tw");
    for (int j : {0, 1, 2, 3, 5, 255, 256, 4097, n / 2 + 7, n - 1})
      std::printf(" %u %u", primeutil::ToMontgomery<word>(pr[j], p),
                  primeutil::ToMontgomery<word>(pir[j], p));
    std::printf("\n");
  }

  // ModSwitch.cu:320-370 table recipe (restore range empty).
  std::vector<word> src(primes.begin(), primes.begin() + ns);
  std::vector<word> dst(primes.begin() + ns, primes.end());
  std::printf("const1");
  for (int i = 0; i < ns; i++) {
    word v = 1;
    for (int j = 0; j < ns; j++)
      if (j != i) v = primeutil::MultMod<word>(v, src[j], src[i]);
    v = primeutil::MultMod<word>(v, static_cast<word>(n), src[i]);
    v = primeutil::InvMod<word>(v, src[i]);
    std::printf(" %u", v);
  }
  std::printf("\nconst2");
  for (int m = 0; m < nd; m++) {
    for (int i = 0; i < ns; i++) {
      word acc = 1;
      for (int j = 0; j < ns; j++)
        if (j != i) acc = primeutil::MultMod<word>(acc, src[j], dst[m]);
      acc = primeutil::ToMontgomery<word>(acc, dst[m]);
      acc = primeutil::ToMontgomery<word>(acc, dst[m]);
      int32_t c = static_cast<int32_t>(acc);
      if (acc > (dst[m] >> 1)) c -= static_cast<int32_t>(dst[m]);
      std::printf(" %d", c);
    }
  }
  std::printf("\ninvpp");
  for (int m = 0; m < nd; m++) {
    word v = 1;
    for (int j = 0; j < ns; j++) v = primeutil::MultMod<word>(v, src[j], dst[m]);
    v = primeutil::InvMod<word>(v, dst[m]);
    std::printf(" %u", primeutil::ToMontgomery<word>(v, dst[m]));
  }
  std::printf("\n");
  return 0;
}
