/*
 * CPU oracle for the CKKS hybrid key-switch hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Plain C99 + unsigned __int128.
 * Citations are to the Cheddar reference tree (include/, src/).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;
typedef __int128 i128;

/* ------------------------------------------------------------------------ */
/* number theory: include/common/PrimeUtils.h                               */
/* ------------------------------------------------------------------------ */

/* PrimeUtils.h:57-61 */
uint32_t orc_mulmod(uint32_t a, uint32_t b, uint32_t q) {
  return (uint32_t)(((uint64_t)a * b) % q);
}

/* PrimeUtils.h:71-83: a^-1 mod q by the extended Euclidean algorithm */
uint32_t orc_invmod(uint32_t a, uint32_t q) {
  int64_t t = 0, nt = 1, r = q, nr = a % q;
  if (nr == 0) return 0;
  while (nr != 0) {
    int64_t quo = r / nr, tmp;
    tmp = t - quo * nt; t = nt; nt = tmp;
    tmp = r - quo * nr; r = nr; nr = tmp;
  }
  if (t < 0) t += q;
  return (uint32_t)t;
}

/* PrimeUtils.h:94-126: exponent taken mod (q-1), negative -> inverse base */
uint32_t orc_powmod(uint32_t a, int64_t e, uint32_t q) {
  a %= q;
  if (a == 0) return 0;
  int64_t m = (int64_t)q - 1;
  e %= m;
  if (e < 0) e += m;
  uint64_t r = 1, b = a;
  uint64_t x = (uint64_t)e;
  while (x) {
    if (x & 1) r = (r * b) % q;
    b = (b * b) % q;
    x >>= 1;
  }
  return (uint32_t)r;
}

/* PrimeUtils.h:135-174: the SMALLEST generator of (Z/q)^* */
uint32_t orc_find_generator(uint32_t q) {
  uint32_t phi = q - 1, temp = phi;
  uint32_t factors[32];
  int nf = 0;
  uint32_t s = (uint32_t)sqrt((double)phi);
  for (uint32_t i = 2; i <= s; i++) {
    if (temp % i == 0) {
      factors[nf++] = i;
      while (temp % i == 0) temp /= i;
      if (temp == 1) break;
    }
  }
  if (temp > 1) factors[nf++] = temp;
  for (uint32_t r = 2; r <= phi; r++) {
    int ok = 1;
    for (int f = 0; f < nf; f++) {
      if (orc_powmod(r, phi / factors[f], q) == 1) { ok = 0; break; }
    }
    if (ok) return r;
  }
  return 0;
}

/* PrimeUtils.h:184-196: g^((q-1)/m) */
uint32_t orc_primitive_root(uint32_t m, uint32_t q) {
  if ((q - 1) % m != 0) return 0;
  return orc_powmod(orc_find_generator(q), (q - 1) / m, q);
}

/* PrimeUtils.h:205-232: q^-1 mod 2^32 read as a signed 32-bit integer */
int32_t orc_inv_mod_base(uint32_t q) {
  uint32_t x = q; /* correct to 3 bits for odd q */
  for (int i = 0; i < 5; i++) x *= 2u - q * x;
  return (int32_t)x;
}

/* PrimeUtils.h:242-248 */
uint32_t orc_to_mont(uint32_t a, uint32_t q) {
  return (uint32_t)((((uint64_t)a) << 32) % q);
}

static uint32_t r_inv(uint32_t q) {
  return orc_invmod((uint32_t)((((uint64_t)1) << 32) % q), q);
}

/* exact canonical a*b*2^-32 mod q */
uint32_t orc_mont_mul(uint32_t a, uint32_t b, uint32_t q) {
  return orc_mulmod(orc_mulmod(a, b, q), r_inv(q), q);
}

/* CommonUtils.h:109-151 */
uint32_t orc_bitrev(uint32_t i, int bits) {
  uint32_t r = 0;
  for (int b = 0; b < bits; b++) r |= ((i >> b) & 1u) << (bits - 1 - b);
  return r;
}

/* ------------------------------------------------------------------------ */
/* kernel-faithful signed lazy Montgomery: include/common/Basic.cuh:72-137  */
/* ------------------------------------------------------------------------ */

/* input a in [-q 2^31, q 2^31), output in (-q, q) */
static inline int32_t mont_reduce_lazy(int64_t a, uint32_t q, int32_t qinv) {
  uint32_t lo = (uint32_t)(uint64_t)a;
  int32_t hi = (int32_t)(a >> 32);
  int32_t t = (int32_t)(lo * (uint32_t)qinv);
  int32_t u = (int32_t)(((int64_t)t * (int64_t)(int32_t)q) >> 32);
  return hi - u;
}

static inline int32_t mont_mul_lazy(int32_t a, int32_t b, uint32_t q,
                                    int32_t qinv) {
  return mont_reduce_lazy((int64_t)a * (int64_t)b, q, qinv);
}

/* ------------------------------------------------------------------------ */
/* twiddles: src/core/NTT.cu:1233-1299                                      */
/* ------------------------------------------------------------------------ */
void orc_twiddles(uint32_t q, int log_n, uint32_t *psi_rev,
                  uint32_t *psi_inv_rev, uint32_t *consts) {
  uint32_t n = 1u << log_n;
  uint32_t g = orc_find_generator(q);
  uint32_t psi = orc_powmod(g, (q - 1) / (2 * n), q);
  uint32_t psi_inv = orc_invmod(psi, q);
  uint64_t p = 1, pi = 1;
  for (uint32_t j = 0; j < n; j++) {
    uint32_t r = orc_bitrev(j, log_n);
    if (psi_rev) psi_rev[r] = orc_to_mont((uint32_t)p, q);
    if (psi_inv_rev) psi_inv_rev[r] = orc_to_mont((uint32_t)pi, q);
    p = (p * psi) % q;
    pi = (pi * psi_inv) % q;
  }
  if (consts) {
    uint32_t ninv = orc_invmod(n % q, q);
    consts[0] = ninv;
    consts[1] = orc_to_mont(ninv, q);
    consts[2] = orc_to_mont(orc_to_mont(1, q), q);
    consts[3] = psi;
    consts[4] = g;
  }
}

/* Twiddle-table cache keyed by (q, log_n) so repeated limb transforms (the
 * CPU baseline) do not rebuild tables; filled under a lock, never evicted
 * beyond its capacity (then tables are built per call). */
#define ORC_CACHE 256
static struct {
  uint32_t q;
  int log_n;
  uint32_t *tw, *itw, c[5];
} g_cache[ORC_CACHE];
static int g_cache_n = 0;

static int cached_tables(uint32_t q, int log_n, const uint32_t **tw,
                         const uint32_t **itw, uint32_t *consts) {
  int hit = -1;
#pragma omp critical(orc_cache)
  {
    for (int i = 0; i < g_cache_n; i++)
      if (g_cache[i].q == q && g_cache[i].log_n == log_n) { hit = i; break; }
    if (hit < 0 && g_cache_n < ORC_CACHE) {
      uint32_t n = 1u << log_n;
      hit = g_cache_n;
      g_cache[hit].tw = (uint32_t *)malloc(sizeof(uint32_t) * n);
      g_cache[hit].itw = (uint32_t *)malloc(sizeof(uint32_t) * n);
      orc_twiddles(q, log_n, g_cache[hit].tw, g_cache[hit].itw, g_cache[hit].c);
      g_cache[hit].q = q;
      g_cache[hit].log_n = log_n;
      g_cache_n++;
    }
  }
  if (hit < 0) return 0;
  *tw = g_cache[hit].tw;
  *itw = g_cache[hit].itw;
  if (consts) memcpy(consts, g_cache[hit].c, sizeof(g_cache[hit].c));
  return 1;
}

/* ------------------------------------------------------------------------ */
/* NTT, kernel-faithful: butterflies NTTUtils.cuh:19-60, structure          */
/* NTT.cu:231-454 (stage order), epilogue NTTUtils.cuh:369-391              */
/* ------------------------------------------------------------------------ */

/* forward CT: twiddle for butterfly group i at stage with m groups is
 * psi_rev[m + i] (NTTUtils.cuh:62-87 index tw_idx << (stage-1)). */
void orc_ntt(uint32_t *x, int log_n, uint32_t q, int mont_conv) {
  uint32_t n = 1u << log_n;
  uint32_t c[5];
  const uint32_t *tw, *itw_unused;
  uint32_t *owned = NULL;
  if (!cached_tables(q, log_n, &tw, &itw_unused, c)) {
    owned = (uint32_t *)malloc(sizeof(uint32_t) * n);
    orc_twiddles(q, log_n, owned, NULL, c);
    tw = owned;
  }
  int32_t qinv = orc_inv_mod_base(q);
  int32_t *a = (int32_t *)x;
  if (mont_conv) {
    for (uint32_t j = 0; j < n; j++) {
      int32_t v = mont_mul_lazy(a[j], (int32_t)c[2], q, qinv);
      a[j] = v;
    }
  }
  uint32_t t = n;
  for (uint32_t m = 1; m < n; m <<= 1) {
    t >>= 1;
    for (uint32_t i = 0; i < m; i++) {
      int32_t w = (int32_t)tw[m + i];
      uint32_t j1 = 2 * i * t;
      for (uint32_t j = j1; j < j1 + t; j++) {
        int32_t u = a[j], v = a[j + t];
        if (u < 0) u += (int32_t)q;
        int32_t mu = mont_mul_lazy(v, w, q, qinv);
        if (mu < 0) mu += (int32_t)q;
        a[j + t] = u - mu;
        a[j] = (u - (int32_t)q) + mu;
      }
    }
  }
  for (uint32_t j = 0; j < n; j++)
    if (a[j] < 0) a[j] += (int32_t)q;
  free(owned);
}

/* GS inverse without the N^-1 factor (kernels compute N * intt) */
static void intt_raw(int32_t *a, int log_n, uint32_t q, const uint32_t *itw,
                     int32_t qinv) {
  uint32_t n = 1u << log_n;
  uint32_t t = 1;
  for (uint32_t m = n >> 1; m >= 1; m >>= 1) {
    for (uint32_t i = 0; i < m; i++) {
      int32_t w = (int32_t)itw[m + i];
      uint32_t j1 = 2 * i * t;
      for (uint32_t j = j1; j < j1 + t; j++) {
        int32_t u = a[j], v = a[j + t];
        if (u < 0) u += (int32_t)q;
        if (v < 0) v += (int32_t)q;
        int32_t d = u - v;
        a[j] = (u - (int32_t)q) + v;
        a[j + t] = mont_mul_lazy(d, w, q, qinv);
      }
    }
    t <<= 1;
  }
}

void orc_intt_mult_const(int32_t *out, const uint32_t *x, int log_n, uint32_t q,
                         uint32_t cst, int normalize) {
  uint32_t n = 1u << log_n;
  const uint32_t *itw, *tw_unused;
  uint32_t *owned = NULL;
  if (!cached_tables(q, log_n, &tw_unused, &itw, NULL)) {
    owned = (uint32_t *)malloc(sizeof(uint32_t) * n);
    orc_twiddles(q, log_n, NULL, owned, NULL);
    itw = owned;
  }
  int32_t qinv = orc_inv_mod_base(q);
  if ((const void *)out != (const void *)x)
    memcpy(out, x, sizeof(uint32_t) * n);
  intt_raw(out, log_n, q, itw, qinv);
  for (uint32_t j = 0; j < n; j++) {
    int32_t v = mont_mul_lazy(out[j], (int32_t)cst, q, qinv);
    if (v < 0) v += (int32_t)q;
    if (normalize && v > (int32_t)(q >> 1)) v -= (int32_t)q;
    out[j] = v;
  }
  free(owned);
}

/* NTT.cu:673-741: epilogue constant N^-1 (mont_conv) or N^-1 R */
void orc_intt(uint32_t *x, int log_n, uint32_t q, int mont_conv) {
  uint32_t n = 1u << log_n;
  uint32_t ninv = orc_invmod(n % q, q);
  uint32_t cst = mont_conv ? ninv : orc_to_mont(ninv, q);
  orc_intt_mult_const((int32_t *)x, x, log_n, q, cst, 0);
}

static int g_threads = 1;

/* CPU-baseline knob: limbs of a batch are spread over this many threads */
void orc_set_threads(int threads) { g_threads = threads > 0 ? threads : 1; }

void orc_ntt_batch(uint32_t *x, int num_limbs, int log_n, const uint32_t *primes,
                   int mont_conv) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int l = 0; l < num_limbs; l++)
    orc_ntt(x + ((size_t)l << log_n), log_n, primes[l], mont_conv);
}

void orc_intt_batch(uint32_t *x, int num_limbs, int log_n,
                    const uint32_t *primes, int mont_conv) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int l = 0; l < num_limbs; l++)
    orc_intt(x + ((size_t)l << log_n), log_n, primes[l], mont_conv);
}

/* ------------------------------------------------------------------------ */
/* NTT, exact canonical arithmetic (independent second path)                 */
/* ------------------------------------------------------------------------ */
void orc_ntt_exact(uint32_t *x, int log_n, uint32_t q, int mont_conv) {
  uint32_t n = 1u << log_n;
  uint32_t *tw = (uint32_t *)malloc(sizeof(uint32_t) * n);
  uint32_t psi = orc_primitive_root(2 * n, q);
  uint64_t p = 1;
  for (uint32_t j = 0; j < n; j++) {
    tw[orc_bitrev(j, log_n)] = (uint32_t)p;
    p = (p * psi) % q;
  }
  if (mont_conv)
    for (uint32_t j = 0; j < n; j++) x[j] = orc_to_mont(x[j] % q, q);
  uint32_t t = n;
  for (uint32_t m = 1; m < n; m <<= 1) {
    t >>= 1;
    for (uint32_t i = 0; i < m; i++) {
      uint64_t w = tw[m + i];
      uint32_t j1 = 2 * i * t;
      for (uint32_t j = j1; j < j1 + t; j++) {
        uint64_t u = x[j], v = (x[j + t] * w) % q;
        x[j] = (uint32_t)((u + v) % q);
        x[j + t] = (uint32_t)((u + q - v) % q);
      }
    }
  }
  free(tw);
}

void orc_intt_exact(uint32_t *x, int log_n, uint32_t q, int mont_conv) {
  uint32_t n = 1u << log_n;
  uint32_t *tw = (uint32_t *)malloc(sizeof(uint32_t) * n);
  uint32_t psi_inv = orc_invmod(orc_primitive_root(2 * n, q), q);
  uint64_t p = 1;
  for (uint32_t j = 0; j < n; j++) {
    tw[orc_bitrev(j, log_n)] = (uint32_t)p;
    p = (p * psi_inv) % q;
  }
  uint32_t t = 1;
  for (uint32_t m = n >> 1; m >= 1; m >>= 1) {
    for (uint32_t i = 0; i < m; i++) {
      uint64_t w = tw[m + i];
      uint32_t j1 = 2 * i * t;
      for (uint32_t j = j1; j < j1 + t; j++) {
        uint64_t u = x[j], v = x[j + t];
        x[j] = (uint32_t)((u + v) % q);
        x[j + t] = (uint32_t)(((u + q - v) % q) * w % q);
      }
    }
    t <<= 1;
  }
  uint64_t s = orc_invmod(n % q, q);
  if (mont_conv) s = (s * r_inv(q)) % q;
  for (uint32_t j = 0; j < n; j++) x[j] = (uint32_t)((x[j] * s) % q);
  free(tw);
}

/* ------------------------------------------------------------------------ */
/* BConv: ModSwitch.cu:23-171 (result is the exact residue; the kernel's    */
/* int64 folding every 4 terms only adds multiples of p 2^32)               */
/* ------------------------------------------------------------------------ */
void orc_bconv(uint32_t *dst, const int32_t *src, int src_len, int dst_len,
               const int32_t *table, const uint32_t *dst_primes, int log_n) {
  size_t n = (size_t)1 << log_n;
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int k = 0; k < dst_len; k++) {
    uint32_t p = dst_primes[k];
    uint64_t ri = r_inv(p);
    const int32_t *row = table + (size_t)k * src_len;
    for (size_t c = 0; c < n; c++) {
      i128 acc = 0;
      for (int i = 0; i < src_len; i++)
        acc += (i128)((int64_t)src[(size_t)i * n + c] * (int64_t)row[i]);
      int64_t r = (int64_t)(acc % (i128)p);
      if (r < 0) r += p;
      dst[(size_t)k * n + c] = (uint32_t)(((uint64_t)r * ri) % p);
    }
  }
}

/* ------------------------------------------------------------------------ */
/* ModSwitch constants: ModSwitch.cu:320-411                                 */
/* ------------------------------------------------------------------------ */
static int32_t normalize(uint32_t a, uint32_t q) {
  int32_t r = (int32_t)a;
  if (a > (q >> 1)) r -= (int32_t)q;
  return r;
}

void orc_modswitch_consts(const uint32_t *src_primes, int src_len,
                          const uint32_t *dst_primes, int dst_len, int log_n,
                          int restore_start, int restore_end, uint32_t *const1,
                          int32_t *const2) {
  uint32_t n = 1u << log_n;
  for (int i = 0; i < src_len; i++) {
    uint32_t m = src_primes[i];
    uint32_t v = 1;
    for (int j = 0; j < src_len; j++)
      if (j != i) v = orc_mulmod(v, src_primes[j], m);
    v = orc_mulmod(v, n, m);
    v = orc_invmod(v, m);
    for (int j = restore_start; j < restore_end; j++)
      v = orc_mulmod(v, dst_primes[j], m);
    const1[i] = v;
  }
  for (int k = 0; k < dst_len; k++) {
    uint32_t m = dst_primes[k];
    for (int i = 0; i < src_len; i++) {
      uint32_t acc = 1;
      for (int j = 0; j < src_len; j++)
        if (j != i) acc = orc_mulmod(acc, src_primes[j], m);
      acc = orc_to_mont(orc_to_mont(acc, m), m);
      const2[(size_t)k * src_len + i] = normalize(acc, m);
    }
  }
}

void orc_moddown_epilogue_consts(const uint32_t *src_primes, int src_len,
                                 const uint32_t *dst_primes, int dst_len,
                                 int restore_start, int restore_end,
                                 uint32_t *inv_prime_prod, uint32_t *padding) {
  int restore_len = restore_end - restore_start;
  for (int i = 0; i < dst_len; i++) {
    uint32_t m = dst_primes[i];
    uint32_t v = 1;
    for (int j = 0; j < src_len; j++) v = orc_mulmod(v, src_primes[j], m);
    inv_prime_prod[i] = orc_to_mont(orc_invmod(v, m), m);
  }
  if (!padding) return;
  for (int i = 0; i < dst_len - restore_len; i++) {
    int idx = i >= restore_start ? i + restore_len : i;
    uint32_t m = dst_primes[idx];
    uint32_t v = 1;
    for (int j = restore_start; j < restore_end; j++)
      v = orc_mulmod(v, dst_primes[j], m);
    padding[i] = orc_to_mont(v, m);
  }
}

/* ------------------------------------------------------------------------ */
/* ModUp: ModSwitch.cu:175-235 (constants) and 429-509 (sequence)           */
/* ------------------------------------------------------------------------ */
int orc_mod_up(uint32_t *dst, const uint32_t *src, int L,
               const uint32_t *q_primes, const uint32_t *p_primes, int alpha,
               int log_n) {
  return orc_mod_up_ex(dst, src, L, q_primes, p_primes, alpha, 0, log_n);
}

/* Groups sit on the full chain's positions (ModSwitch.cu:200-235, 429-509):
 * with prime_offset = max_ter - num_ter missing terminal primes in front,
 * group g covers the level's limbs [max(0, g alpha - off),
 * min((g+1) alpha, L + off) - off); groups that end at or before off are
 * empty and left untouched in dst. */
int orc_mod_up_ex(uint32_t *dst, const uint32_t *src, int L,
                  const uint32_t *q_primes, const uint32_t *p_primes,
                  int alpha, int prime_offset, int log_n) {
  size_t n = (size_t)1 << log_n;
  int total = L + alpha;
  int beta = (L + prime_offset + alpha - 1) / alpha;
  uint32_t *primes = (uint32_t *)malloc(sizeof(uint32_t) * total);
  memcpy(primes, q_primes, sizeof(uint32_t) * L);
  memcpy(primes + L, p_primes, sizeof(uint32_t) * alpha);
  int32_t *centred = (int32_t *)malloc(sizeof(int32_t) * n * L);
  uint32_t *const1 = (uint32_t *)malloc(sizeof(uint32_t) * alpha);
  int32_t *const2 = (int32_t *)malloc(sizeof(int32_t) * alpha * total);
  uint32_t *dprimes = (uint32_t *)malloc(sizeof(uint32_t) * total);
  uint32_t *z = (uint32_t *)malloc(sizeof(uint32_t) * n * total);
  for (int g = 0; g < beta; g++) {
    int abs_end = (g + 1) * alpha < L + prime_offset ? (g + 1) * alpha
                                                     : L + prime_offset;
    if (abs_end <= prime_offset) continue;
    int start = g * alpha - prime_offset > 0 ? g * alpha - prime_offset : 0;
    int end = abs_end - prime_offset;
    int slen = end - start;
    int dlen = total - slen;
    for (int k = 0; k < start; k++) dprimes[k] = primes[k];
    for (int k = end; k < total; k++) dprimes[k - slen] = primes[k];
    orc_modswitch_consts(primes + start, slen, dprimes, dlen, log_n, 0, 0,
                         const1, const2);
    /* INTTAndMultConst(normalize) over the group's own limbs */
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int i = 0; i < slen; i++)
      orc_intt_mult_const(centred + (size_t)(start + i) * n,
                          src + (size_t)(start + i) * n, log_n,
                          primes[start + i], const1[i], 1);
    orc_bconv(z, centred + (size_t)start * n, slen, dlen, const2, dprimes,
              log_n);
    uint32_t *out = dst + (size_t)g * total * n;
    memcpy(out + (size_t)start * n, src + (size_t)start * n,
           sizeof(uint32_t) * n * slen);
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int k = 0; k < dlen; k++) {
      int pos = k < start ? k : k + slen;
      uint32_t *limb = out + (size_t)pos * n;
      memcpy(limb, z + (size_t)k * n, sizeof(uint32_t) * n);
      orc_ntt(limb, log_n, primes[pos], 0);
    }
  }
  free(primes); free(centred); free(const1); free(const2); free(dprimes);
  free(z);
  return beta;
}

/* ------------------------------------------------------------------------ */
/* ModDown family: ModSwitch.cu:566-684, epilogue NTT.cu:456-601            */
/* ------------------------------------------------------------------------ */
void orc_mod_down(uint32_t *dst, const uint32_t *src, int src_total,
                  const uint32_t *src_primes, int dst_len, int log_n) {
  int slen = src_total - dst_len;
  int *drop = (int *)malloc(sizeof(int) * (slen > 0 ? slen : 1));
  int *dsrc = (int *)malloc(sizeof(int) * (dst_len > 0 ? dst_len : 1));
  for (int i = 0; i < slen; i++) drop[i] = dst_len + i;
  for (int k = 0; k < dst_len; k++) dsrc[k] = k;
  orc_mod_down_ex(dst, src, src_primes, drop, slen, src_primes, dst_len, dsrc,
                  log_n);
  free(drop); free(dsrc);
}

/* The general form with the BitPacker restore (ModSwitch.cu:258-411, 566-684;
 * NTT.cu:456-601, 1073-1127): the source limbs drop[0..num_drop) are divided
 * out; destination limb k has primes dst_primes[k] and takes its kept value
 * from source limb dst_src[k], or, when dst_src[k] < 0, is a restored prime
 * with no source limb. With R the product of the restored primes:
 *   c_i  = centre(INTT(src_i) (N prod_{j != i} q_j)^-1 R)        (i in drop)
 *   z_k  = R sum_i c_i prod_{j != i} q_j mod p_k  (BConv, double Montgomery)
 *   dst_k = MontMul(MontMul(src[dst_src[k]], ToMont(R)) - NTT(z_k),
 *                   ToMont((prod_{i in drop} q_i)^-1))
 * and for restored limbs the src term is 0. */
void orc_mod_down_ex(uint32_t *dst, const uint32_t *src,
                     const uint32_t *src_primes, const int *drop, int num_drop,
                     const uint32_t *dst_primes, int dst_len,
                     const int *dst_src, int log_n) {
  size_t n = (size_t)1 << log_n;
  int slen = num_drop;
  uint32_t *sp = (uint32_t *)malloc(sizeof(uint32_t) * (slen > 0 ? slen : 1));
  for (int i = 0; i < slen; i++) sp[i] = src_primes[drop[i]];
  uint32_t *const1 = (uint32_t *)malloc(sizeof(uint32_t) * (slen > 0 ? slen : 1));
  int32_t *const2 = (int32_t *)malloc(sizeof(int32_t) * (slen > 0 ? slen : 1) * dst_len);
  int32_t *centred = (int32_t *)malloc(sizeof(int32_t) * n * (slen > 0 ? slen : 1));
  uint32_t *z = (uint32_t *)malloc(sizeof(uint32_t) * n * dst_len);
  for (int i = 0; i < slen; i++) {
    uint32_t m = sp[i], v = 1;
    for (int j = 0; j < slen; j++)
      if (j != i) v = orc_mulmod(v, sp[j], m);
    v = orc_mulmod(v, (uint32_t)n, m);
    v = orc_invmod(v, m);
    for (int k = 0; k < dst_len; k++)
      if (dst_src[k] < 0) v = orc_mulmod(v, dst_primes[k], m);
    const1[i] = v;
  }
  for (int k = 0; k < dst_len; k++) {
    uint32_t m = dst_primes[k];
    for (int i = 0; i < slen; i++) {
      uint32_t acc = 1;
      for (int j = 0; j < slen; j++)
        if (j != i) acc = orc_mulmod(acc, sp[j], m);
      acc = orc_to_mont(orc_to_mont(acc, m), m);
      const2[(size_t)k * slen + i] = normalize(acc, m);
    }
  }
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int i = 0; i < slen; i++)
    orc_intt_mult_const(centred + (size_t)i * n, src + (size_t)drop[i] * n,
                        log_n, sp[i], const1[i], 1);
  orc_bconv(z, centred, slen, dst_len, const2, dst_primes, log_n);
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int k = 0; k < dst_len; k++) {
    uint32_t q = dst_primes[k];
    uint32_t inv = 1, pad = 1;
    for (int i = 0; i < slen; i++) inv = orc_mulmod(inv, sp[i] % q, q);
    inv = orc_to_mont(orc_invmod(inv, q), q);
    for (int j = 0; j < dst_len; j++)
      if (dst_src[j] < 0) pad = orc_mulmod(pad, dst_primes[j] % q, q);
    pad = orc_to_mont(pad, q);
    uint32_t *zl = z + (size_t)k * n;
    orc_ntt(zl, log_n, q, 0);
    uint32_t *o = dst + (size_t)k * n;
    const uint32_t *s = dst_src[k] >= 0 ? src + (size_t)dst_src[k] * n : NULL;
    for (size_t c = 0; c < n; c++) {
      uint32_t v = s ? orc_mont_mul(s[c] % q, pad, q) : 0;
      uint32_t d = v >= zl[c] ? v - zl[c] : v + q - zl[c];
      o[c] = orc_mont_mul(d, inv, q);
    }
  }
  free(sp); free(const1); free(const2); free(centred); free(z);
}

/* ------------------------------------------------------------------------ */
/* element-wise: ElementWise.cu                                              */
/* ------------------------------------------------------------------------ */

/* Tensor (ElementWise.cu:504-546): Karatsuba in Montgomery form */
void orc_tensor(uint32_t *bx, uint32_t *ax, uint32_t *rx, const uint32_t *b1,
                const uint32_t *a1, const uint32_t *b2, const uint32_t *a2,
                int num_limbs, const uint32_t *primes, int log_n) {
  size_t n = (size_t)1 << log_n;
  for (int l = 0; l < num_limbs; l++) {
    uint32_t q = primes[l];
    uint64_t ri = r_inv(q);
    for (size_t c = 0; c < n; c++) {
      size_t i = (size_t)l * n + c;
      uint64_t bb = ((uint64_t)b1[i] * b2[i]) % q * ri % q;
      uint64_t aa = ((uint64_t)a1[i] * a2[i]) % q * ri % q;
      uint64_t s1 = ((uint64_t)b1[i] + a1[i]) % q;
      uint64_t s2 = ((uint64_t)b2[i] + a2[i]) % q;
      uint64_t mid = (s1 * s2) % q * ri % q;
      mid = (mid + 2 * (uint64_t)q - bb - aa) % q;
      bx[i] = (uint32_t)bb;
      ax[i] = (uint32_t)mid;
      rx[i] = (uint32_t)aa;
    }
  }
}

/* PAccum (ElementWise.cu:225-287, Context.cpp:609-647) */
void orc_paccum(uint32_t *acc_b, uint32_t *acc_a, const uint32_t *modup,
                int beta, const uint32_t *key_b, const uint32_t *key_a, int L,
                int alpha, int max_q, const uint32_t *primes, int log_n) {
  size_t n = (size_t)1 << log_n;
  int total = L + alpha;
  size_t key_stride = (size_t)(max_q + alpha) * n;
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int l = 0; l < total; l++) {
    uint32_t q = primes[l];
    uint64_t ri = r_inv(q);
    int kl = l < L ? l : max_q + (l - L);
    for (size_t c = 0; c < n; c++) {
      uint64_t sb = 0, sa = 0;
      for (int g = 0; g < beta; g++) {
        uint64_t m = modup[(size_t)g * total * n + (size_t)l * n + c];
        sb += m * key_b[g * key_stride + (size_t)kl * n + c] % q;
        sa += m * key_a[g * key_stride + (size_t)kl * n + c] % q;
      }
      acc_b[(size_t)l * n + c] = (uint32_t)((sb % q) * ri % q);
      acc_a[(size_t)l * n + c] = (uint32_t)((sa % q) * ri % q);
    }
  }
}

/* PAccum over the non-empty groups of a ModUp with a prime offset
 * (Context.cpp:609-647): modup group j is paired with key group key_group[j];
 * q limb l reads key limb key_off + l, aux limb L + k reads max_q + k. */
void orc_paccum_ex(uint32_t *acc_b, uint32_t *acc_a, const uint32_t *modup,
                   int num_groups, const int *key_group, const uint32_t *key_b,
                   const uint32_t *key_a, int L, int alpha, int max_q,
                   int key_off, const uint32_t *primes, int log_n) {
  size_t n = (size_t)1 << log_n;
  int total = L + alpha;
  size_t key_stride = (size_t)(max_q + alpha) * n;
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int l = 0; l < total; l++) {
    uint32_t q = primes[l];
    uint64_t ri = r_inv(q);
    int kl = l < L ? key_off + l : max_q + (l - L);
    for (size_t c = 0; c < n; c++) {
      uint64_t sb = 0, sa = 0;
      for (int j = 0; j < num_groups; j++) {
        size_t ko = (size_t)key_group[j] * key_stride + (size_t)kl * n + c;
        uint64_t m = modup[(size_t)j * total * n + (size_t)l * n + c];
        sb += m * key_b[ko] % q;
        sa += m * key_a[ko] % q;
      }
      acc_b[(size_t)l * n + c] = (uint32_t)((sb % q) * ri % q);
      acc_a[(size_t)l * n + c] = (uint32_t)((sa % q) * ri % q);
    }
  }
}

/* CAccum (ElementWise.cu:291-366, Context.cpp:684-699) */
void orc_caccum(uint32_t *acc, const uint32_t *ct, const uint32_t *p_prod,
                int L, const uint32_t *primes, int log_n) {
  size_t n = (size_t)1 << log_n;
  for (int l = 0; l < L; l++) {
    uint32_t q = primes[l];
    uint64_t ri = r_inv(q);
    for (size_t c = 0; c < n; c++) {
      size_t i = (size_t)l * n + c;
      uint64_t m = (uint64_t)p_prod[l] * ct[i] % q * ri % q;
      acc[i] = (uint32_t)((acc[i] + m) % q);
    }
  }
}

/* GSFusedKernel (Hoist.cu:80-118): the giant-step accumulator gains
 * MontMul(plaintext, baby step) per (giant, baby) pair, canonical sums */
void orc_pmult_accum(uint32_t *acc, const uint32_t *pt, const uint32_t *x,
                     int num_limbs, const uint32_t *primes, int log_n) {
  size_t n = (size_t)1 << log_n;
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int l = 0; l < num_limbs; l++) {
    uint32_t q = primes[l];
    uint64_t ri = r_inv(q);
    for (size_t c = 0; c < n; c++) {
      size_t i = (size_t)l * n + c;
      uint64_t m = (uint64_t)pt[i] * x[i] % q * ri % q;
      acc[i] = (uint32_t)((acc[i] + m) % q);
    }
  }
}

void orc_p_prod(uint32_t *p_prod, const uint32_t *q_primes, int L,
                const uint32_t *p_primes, int alpha) {
  for (int l = 0; l < L; l++) {
    uint32_t v = 1;
    for (int j = 0; j < alpha; j++) v = orc_mulmod(v, p_primes[j], q_primes[l]);
    p_prod[l] = orc_to_mont(v, q_primes[l]);
  }
}

/* Permute (ElementWise.cu:370-391) */
void orc_permute(uint32_t *dst, const uint32_t *src, int num_limbs, int log_n,
                 uint32_t galois) {
  size_t n = (size_t)1 << log_n;
  uint32_t mask = (uint32_t)(2 * n - 1);
#pragma omp parallel for num_threads(g_threads) schedule(static)
  for (int l = 0; l < num_limbs; l++) {
    for (size_t x = 0; x < n; x++) {
      uint32_t e = orc_bitrev((uint32_t)x, log_n + 1) + 1;
      uint32_t s = orc_bitrev((e * galois - 1) & mask, log_n + 1);
      dst[(size_t)l * n + x] = src[(size_t)l * n + s];
    }
  }
}

/* Parameter.cu:93-101 and ElementWise.cu:955-964 */
uint32_t orc_galois_factor(int rot, int log_n) {
  uint32_t m = 2u << log_n;
  if (rot == -1) return m - 1;
  uint32_t g = 1;
  int half = 1 << (log_n - 1);
  if (rot == half) return 1;
  for (int i = 0; i < rot; i++) g = (uint32_t)(((uint64_t)g * 5) % m);
  return g;
}

/* ------------------------------------------------------------------------ */
/* key-switch compositions: Context.cpp                                     */
/* ------------------------------------------------------------------------ */
static uint32_t *level_primes(const uint32_t *q, int L, const uint32_t *p,
                              int alpha) {
  uint32_t *pr = (uint32_t *)malloc(sizeof(uint32_t) * (L + alpha));
  memcpy(pr, q, sizeof(uint32_t) * L);
  memcpy(pr + L, p, sizeof(uint32_t) * alpha);
  return pr;
}

/* MultKeyNoModDown (Context.cpp:649-712) on the polynomial d with the extra
 * ct parts: acc_b gets + p_prod * cb, acc_a gets + p_prod * ca when ca. */
static int key_mult_no_mod_down(uint32_t *acc_b, uint32_t *acc_a,
                                const uint32_t *d, const uint32_t *cb,
                                const uint32_t *ca, const uint32_t *key_b,
                                const uint32_t *key_a, int L, int max_q,
                                const uint32_t *q_primes,
                                const uint32_t *p_primes, int alpha,
                                int log_n) {
  size_t n = (size_t)1 << log_n;
  int total = L + alpha;
  int beta = (L + alpha - 1) / alpha;
  uint32_t *pr = level_primes(q_primes, L, p_primes, alpha);
  uint32_t *modup = (uint32_t *)malloc(sizeof(uint32_t) * n * total * beta);
  uint32_t *pp = (uint32_t *)malloc(sizeof(uint32_t) * L);
  orc_mod_up(modup, d, L, q_primes, p_primes, alpha, log_n);
  orc_paccum(acc_b, acc_a, modup, beta, key_b, key_a, L, alpha, max_q, pr,
             log_n);
  orc_p_prod(pp, q_primes, L, p_primes, alpha);
  orc_caccum(acc_b, cb, pp, L, pr, log_n);
  if (ca) orc_caccum(acc_a, ca, pp, L, pr, log_n);
  free(pr); free(modup); free(pp);
  return beta;
}

/* HMult (Context.cpp:862-871) = Tensor + RelinearizeRescale (714-737) or
 * Relinearize (559-562). rescale = number of q primes dropped (0: none). */
int orc_hmult(uint32_t *res_b, uint32_t *res_a, const uint32_t *b1,
              const uint32_t *a1, const uint32_t *b2, const uint32_t *a2,
              const uint32_t *key_b, const uint32_t *key_a, int L, int max_q,
              const uint32_t *q_primes, const uint32_t *p_primes, int alpha,
              int log_n, int rescale) {
  size_t n = (size_t)1 << log_n;
  int total = L + alpha;
  uint32_t *pr = level_primes(q_primes, L, p_primes, alpha);
  uint32_t *bx = (uint32_t *)malloc(sizeof(uint32_t) * n * L);
  uint32_t *ax = (uint32_t *)malloc(sizeof(uint32_t) * n * L);
  uint32_t *rx = (uint32_t *)malloc(sizeof(uint32_t) * n * L);
  uint32_t *acc_b = (uint32_t *)malloc(sizeof(uint32_t) * n * total);
  uint32_t *acc_a = (uint32_t *)malloc(sizeof(uint32_t) * n * total);
  orc_tensor(bx, ax, rx, b1, a1, b2, a2, L, pr, log_n);
  key_mult_no_mod_down(acc_b, acc_a, rx, bx, ax, key_b, key_a, L, max_q,
                       q_primes, p_primes, alpha, log_n);
  orc_mod_down(res_b, acc_b, total, pr, L - rescale, log_n);
  orc_mod_down(res_a, acc_a, total, pr, L - rescale, log_n);
  free(pr); free(bx); free(ax); free(rx); free(acc_b); free(acc_a);
  return 0;
}

/* Rescale (Context.cpp:739-774) of one polynomial */
int orc_rescale(uint32_t *res, const uint32_t *src, int L,
                const uint32_t *q_primes, int drop, int log_n) {
  orc_mod_down(res, src, L, q_primes, L - drop, log_n);
  return 0;
}

/* MultKey (Context.cpp:584-607) */
int orc_mult_key(uint32_t *res_b, uint32_t *res_a, const uint32_t *b,
                 const uint32_t *a, const uint32_t *key_b,
                 const uint32_t *key_a, int L, int max_q,
                 const uint32_t *q_primes, const uint32_t *p_primes, int alpha,
                 int log_n) {
  size_t n = (size_t)1 << log_n;
  int total = L + alpha;
  uint32_t *pr = level_primes(q_primes, L, p_primes, alpha);
  uint32_t *acc_b = (uint32_t *)malloc(sizeof(uint32_t) * n * total);
  uint32_t *acc_a = (uint32_t *)malloc(sizeof(uint32_t) * n * total);
  key_mult_no_mod_down(acc_b, acc_a, a, b, NULL, key_b, key_a, L, max_q,
                       q_primes, p_primes, alpha, log_n);
  orc_mod_down(res_b, acc_b, total, pr, L, log_n);
  orc_mod_down(res_a, acc_a, total, pr, L, log_n);
  free(pr); free(acc_b); free(acc_a);
  return 0;
}

/* HRot (Context.cpp:776-791): key switch first, then permute */
int orc_hrot(uint32_t *res_b, uint32_t *res_a, const uint32_t *b,
             const uint32_t *a, const uint32_t *key_b, const uint32_t *key_a,
             int L, int max_q, const uint32_t *q_primes,
             const uint32_t *p_primes, int alpha, int log_n, int rot) {
  size_t n = (size_t)1 << log_n;
  uint32_t *tb = (uint32_t *)malloc(sizeof(uint32_t) * n * L);
  uint32_t *ta = (uint32_t *)malloc(sizeof(uint32_t) * n * L);
  orc_mult_key(tb, ta, b, a, key_b, key_a, L, max_q, q_primes, p_primes, alpha,
               log_n);
  uint32_t g = orc_galois_factor(rot, log_n);
  orc_permute(res_b, tb, L, log_n, g);
  orc_permute(res_a, ta, L, log_n, g);
  free(tb); free(ta);
  return 0;
}
