// Device-side modular arithmetic for u32 RNS residues (primes q < 2^31).
//
// Two families:
//  * fp64 exact reductions (reduce_f64, centre_f64, mulmod_f64): BConv's
//    recombination of exact integer sums below 2^50. mulmod_f64 forms b*w
//    mod q from h = b*w, l = fma(b,w,-h) (exact low part),
//    t = rint(b*(w/q)), r = fma(-t,q,h) + l: |b| < 2^45 and w < 2^31 keep
//    |h - t*q| < 2^34, an integer, so the fma and the add are exact.
//  * signed Montgomery (R = 2^32) on VALU integers, the reference's
//    convention MontMul(a,b) = a*b*2^-32 mod q
//    (include/common/Basic.cuh:72-137): the NTT and element-wise kernels.
//    gfx950 issues 32-bit mul_lo / mul_hi at about the rate of other 32-bit
//    VALU ops (measured), so three multiplies per product are cheap.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace chd {

constexpr int kLogN = 16;
constexpr int kN = 1 << kLogN;

// ---------------------------------------------------------------- fp64 ----
__device__ __forceinline__ double mulmod_f64(double b, double w, double wq,
                                             double q) {
  double h = b * w;
  double l = __builtin_fma(b, w, -h);
  double t = __builtin_rint(b * wq);
  double r = __builtin_fma(-t, q, h);
  return r + l;
}

// x (|x| < 2^50) -> canonical [0, q) as u32
__device__ __forceinline__ uint32_t reduce_f64(double x, double q,
                                               double qinv) {
  double t = __builtin_rint(x * qinv);
  double r = __builtin_fma(-t, q, x);  // exact, |r| <= q/2 + 1
  int32_t v = static_cast<int32_t>(r);
  uint32_t u = static_cast<uint32_t>(v);
  uint32_t uq = u + static_cast<uint32_t>(q);
  return u < uq ? u : uq;  // unsigned min: picks u + q when v < 0
}

// x -> centred [-(q-1)/2, (q-1)/2] as i32 (q odd)
__device__ __forceinline__ int32_t centre_f64(double x, double q,
                                              double qinv) {
  double t = __builtin_rint(x * qinv);
  double r = __builtin_fma(-t, q, x);  // |r| <= q/2 + 1
  double half = 0.5 * q;               // (q-1)/2 < half < (q+1)/2
  r = r > half ? r - q : r;
  r = r < -half ? r + q : r;
  return static_cast<int32_t>(r);
}

// -------------------------------------------------------- Montgomery ----
__device__ __forceinline__ int32_t mont_reduce_lazy(int64_t a, uint32_t q,
                                                    int32_t qinv) {
  uint32_t lo = static_cast<uint32_t>(a);
  int32_t hi = static_cast<int32_t>(a >> 32);
  int32_t t = static_cast<int32_t>(lo * static_cast<uint32_t>(qinv));
  int32_t u = __mulhi(t, static_cast<int32_t>(q));
  return hi - u;
}

// canonical a*b*2^-32 mod q for a, b in (-2^31, 2^31) with |a*b| < q 2^31
__device__ __forceinline__ uint32_t mont_mul(int32_t a, int32_t b, uint32_t q,
                                             int32_t qinv) {
  int32_t r = mont_reduce_lazy(static_cast<int64_t>(a) * b, q, qinv);
  return static_cast<uint32_t>(r < 0 ? r + static_cast<int32_t>(q) : r);
}

__device__ __forceinline__ uint32_t add_mod(uint32_t a, uint32_t b,
                                            uint32_t q) {
  uint32_t s = a + b;
  uint32_t t = s - q;
  return s < t ? s : t;  // both < 2^32 since q < 2^31
}

__device__ __forceinline__ uint32_t sub_mod(uint32_t a, uint32_t b,
                                            uint32_t q) {
  uint32_t d = a - b;
  uint32_t e = d + q;
  return d < e ? d : e;
}

// sum of up to four products of canonical residues (each < q^2 < 2^62, so
// the sum fits 64 bits) times 2^-32 mod q, canonical: with T = hi 2^32 + lo,
// T 2^-32 = hi + lo 2^-32 (mod q), where hi < 4 q^2 / 2^32 < 2q and the
// Montgomery reduction of lo is in [0, q]. qn = -q^-1 mod 2^32.
__device__ __forceinline__ uint32_t reduce_sum4(uint64_t t, uint32_t q,
                                                uint32_t qn) {
  const uint32_t lo = static_cast<uint32_t>(t);
  uint32_t hi = static_cast<uint32_t>(t >> 32);
  hi = hi < q ? hi : hi - q;                       // [0, q)
  const uint32_t m = lo * qn;
  const uint32_t r = static_cast<uint32_t>(
      (static_cast<uint64_t>(m) * q + lo) >> 32);  // [0, q]
  const uint32_t s = hi + r;                       // [0, 2q)
  return s < q ? s : s - q;
}

// ModUp dnum groups sit on the chain's positions: a level missing `shift`
// limbs of its first group owns limbs [lo, hi) in group g
// (ModSwitch.cu:440-470 with prime_offset mod alpha)
__host__ __device__ __forceinline__ int group_lo(int g, int alpha, int shift) {
  const int v = g * alpha - shift;
  return v > 0 ? v : 0;
}
__host__ __device__ __forceinline__ int group_hi(int g, int alpha, int shift,
                                                 int num_q) {
  const int v = (g + 1) * alpha - shift;
  return v < num_q ? v : num_q;
}
// groups 0..beta-1 cover [0, num_q) and none is empty
inline bool groups_valid(int beta, int alpha, int shift, int num_q) {
  return alpha >= 1 && shift >= 0 && shift < alpha && beta >= 1 &&
         (beta - 1) * alpha - shift < num_q && beta * alpha - shift >= num_q;
}

// wave-uniform value into an SGPR
__device__ __forceinline__ int uniform(int v) {
  return __builtin_amdgcn_readfirstlane(v);
}

}  // namespace chd
