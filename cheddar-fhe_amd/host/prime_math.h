// Host number theory for the constant tables (u32 primes q < 2^31).
//
// Same definitions as the reference's primeutil namespace
// (include/common/PrimeUtils.h:57-248): the NTT root is psi = g^((q-1)/2N)
// with g the SMALLEST generator, q^-1 mod 2^32 is read as a signed 32-bit
// value, ToMontgomery(a) = a * 2^32 mod q. Written independently here.
#pragma once

#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <vector>

namespace cheddar {
namespace pm {

inline uint32_t mulmod(uint32_t a, uint32_t b, uint32_t q) {
  return static_cast<uint32_t>((static_cast<uint64_t>(a) * b) % q);
}

inline uint32_t powmod(uint32_t a, int64_t e, uint32_t q) {
  a %= q;
  if (a == 0) return 0;
  int64_t m = static_cast<int64_t>(q) - 1;
  e %= m;
  if (e < 0) e += m;
  uint64_t r = 1, b = a;
  for (uint64_t x = static_cast<uint64_t>(e); x; x >>= 1) {
    if (x & 1) r = r * b % q;
    b = b * b % q;
  }
  return static_cast<uint32_t>(r);
}

inline uint32_t invmod(uint32_t a, uint32_t q) {
  int64_t t = 0, nt = 1, r = q, nr = a % q;
  if (nr == 0) throw std::invalid_argument("invmod: zero has no inverse");
  while (nr != 0) {
    int64_t quo = r / nr, tmp = t - quo * nt;
    t = nt;
    nt = tmp;
    tmp = r - quo * nr;
    r = nr;
    nr = tmp;
  }
  if (t < 0) t += q;
  return static_cast<uint32_t>(t);
}

inline uint32_t find_generator(uint32_t q) {
  uint32_t phi = q - 1, rest = phi;
  std::vector<uint32_t> factors;
  for (uint32_t i = 2; static_cast<uint64_t>(i) * i <= rest; i++) {
    if (rest % i == 0) {
      factors.push_back(i);
      while (rest % i == 0) rest /= i;
    }
  }
  if (rest > 1) factors.push_back(rest);
  for (uint32_t r = 2; r < q; r++) {
    bool ok = true;
    for (uint32_t f : factors)
      if (powmod(r, phi / f, q) == 1) {
        ok = false;
        break;
      }
    if (ok) return r;
  }
  throw std::runtime_error("find_generator: no generator");
}

inline uint32_t primitive_root(uint32_t m, uint32_t q) {
  if ((q - 1) % m != 0)
    throw std::invalid_argument("prime is not NTT-friendly");
  return powmod(find_generator(q), (q - 1) / m, q);
}

inline int32_t inv_mod_base(uint32_t q) {
  uint32_t x = q;
  for (int i = 0; i < 5; i++) x *= 2u - q * x;
  return static_cast<int32_t>(x);
}

inline uint32_t to_mont(uint32_t a, uint32_t q) {
  return static_cast<uint32_t>((static_cast<uint64_t>(a) << 32) % q);
}

inline int32_t normalize(uint32_t a, uint32_t q) {
  int32_t r = static_cast<int32_t>(a);
  if (a > (q >> 1)) r -= static_cast<int32_t>(q);
  return r;
}

inline uint32_t bitrev(uint32_t i, int bits) {
  uint32_t r = 0;
  for (int b = 0; b < bits; b++) r |= ((i >> b) & 1u) << (bits - 1 - b);
  return r;
}

// Base-conversion constants from the source primes to the destination
// primes (PopulateModSwitchConstants, ModSwitch.cu:320-370), degree n:
//   const1[i]    = (n prod_{j != i} s_j)^-1 mod s_i, times the product of
//                  the restored destination primes [restore_lo, restore_hi)
//                  (BitPacker, ModSwitch.cu:372-411), plain residues;
//   const2[k][i] = centre(ToMont(ToMont(prod_{j != i} s_j mod d_k))), the
//                  "double Montgomery" table of the matrix product.
inline void modswitch_constants(const std::vector<uint32_t> &src,
                                const std::vector<uint32_t> &dst, uint32_t n,
                                int restore_lo, int restore_hi,
                                std::vector<uint32_t> *const1,
                                std::vector<int32_t> *const2) {
  const size_t sl = src.size(), dl = dst.size();
  const1->assign(sl, 1);
  const2->assign(sl * dl, 0);
  for (size_t i = 0; i < sl; i++) {
    uint32_t v = 1;
    for (size_t j = 0; j < sl; j++)
      if (j != i) v = mulmod(v, src[j] % src[i], src[i]);
    v = mulmod(v, n % src[i], src[i]);
    (*const1)[i] = invmod(v, src[i]);
    for (int j = restore_lo; j < restore_hi; j++)
      (*const1)[i] = mulmod((*const1)[i], dst[j] % src[i], src[i]);
  }
  for (size_t k = 0; k < dl; k++)
    for (size_t i = 0; i < sl; i++) {
      uint32_t acc = 1;
      for (size_t j = 0; j < sl; j++)
        if (j != i) acc = mulmod(acc, src[j] % dst[k], dst[k]);
      acc = to_mont(to_mont(acc, dst[k]), dst[k]);
      (*const2)[k * sl + i] = normalize(acc, dst[k]);
    }
}

}  // namespace pm
}  // namespace cheddar
