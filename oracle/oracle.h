/*
 * CPU oracle for the CKKS hybrid key-switch hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP
 * product path is compared against. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product library never links
 * or calls it.
 *
 * Every function is a plain restatement of the reference algorithm with
 * R = 2^32 Montgomery arithmetic on u32 residues (primes q < 2^31).
 * Each definition cites the reference file:line it follows
 * (paths relative to the Cheddar source tree).
 *
 * Two independent NTT paths are kept on purpose:
 *   - orc_ntt / orc_intt_* : kernel-faithful signed lazy Montgomery
 *     butterflies (include/core/NTTUtils.cuh:19-60, Basic.cuh:72-137),
 *   - orc_ntt_exact / orc_intt_exact : canonical arithmetic with `%`.
 * The tests require them to agree, and pin the exact path to the closed-form
 * DFT y[i] = sum_j x_j psi^{(2 brev(i)+1) j}.
 */
#ifndef CHEDDAR_ORACLE_H
#define CHEDDAR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number theory: include/common/PrimeUtils.h:57-248 ---- */
uint32_t orc_mulmod(uint32_t a, uint32_t b, uint32_t q);
uint32_t orc_powmod(uint32_t a, int64_t e, uint32_t q);
uint32_t orc_invmod(uint32_t a, uint32_t q);
uint32_t orc_find_generator(uint32_t q);
uint32_t orc_primitive_root(uint32_t m, uint32_t q);
int32_t orc_inv_mod_base(uint32_t q);
uint32_t orc_to_mont(uint32_t a, uint32_t q);
uint32_t orc_mont_mul(uint32_t a, uint32_t b, uint32_t q);
uint32_t orc_bitrev(uint32_t i, int bits);

/* ---- twiddle tables: src/core/NTT.cu:1233-1299 ----
 * psi_rev[j] = ToMont(psi^brev(j)), psi_inv_rev[j] = ToMont(psi^-brev(j)).
 * consts[0..4] = N^-1, ToMont(N^-1), R^2 mod q, psi, smallest generator g. */
void orc_twiddles(uint32_t q, int log_n, uint32_t *psi_rev,
                  uint32_t *psi_inv_rev, uint32_t *consts);

/* ---- NTT (NTT.cu:606-741) ---- */
/* forward, natural -> bit-reversed; mont_conv multiplies the input by R */
void orc_ntt(uint32_t *x, int log_n, uint32_t q, int mont_conv);
void orc_ntt_exact(uint32_t *x, int log_n, uint32_t q, int mont_conv);
/* inverse with N^-1 folded: mont_conv=1 -> intt * R^-1, 0 -> exact intt */
void orc_intt(uint32_t *x, int log_n, uint32_t q, int mont_conv);
void orc_intt_exact(uint32_t *x, int log_n, uint32_t q, int mont_conv);
/* out = MontMul(N * intt(x), c), centred into [-(q-1)/2,(q-1)/2] when
 * normalize (NTT.cu:743-813, NTTUtils.cuh:369-391). out may alias x. */
void orc_intt_mult_const(int32_t *out, const uint32_t *x, int log_n, uint32_t q,
                         uint32_t c, int normalize);
/* limb-major batches [num_limbs][N], limb i uses primes[i]; limbs are
 * spread over orc_set_threads() OpenMP threads (default 1) */
void orc_set_threads(int threads);
void orc_ntt_batch(uint32_t *x, int num_limbs, int log_n, const uint32_t *primes,
                   int mont_conv);
void orc_intt_batch(uint32_t *x, int num_limbs, int log_n,
                    const uint32_t *primes, int mont_conv);

/* ---- BConv (ModSwitch.cu:23-171) ----
 * dst[k][n] = (sum_i src[i][n] * table[k][i]) * R^-1 mod dst_primes[k]. */
void orc_bconv(uint32_t *dst, const int32_t *src, int src_len, int dst_len,
               const int32_t *table, const uint32_t *dst_primes, int log_n);

/* ---- ModSwitch constants (ModSwitch.cu:320-411) ---- */
void orc_modswitch_consts(const uint32_t *src_primes, int src_len,
                          const uint32_t *dst_primes, int dst_len, int log_n,
                          int restore_start, int restore_end, uint32_t *const1,
                          int32_t *const2);
void orc_moddown_epilogue_consts(const uint32_t *src_primes, int src_len,
                                 const uint32_t *dst_primes, int dst_len,
                                 int restore_start, int restore_end,
                                 uint32_t *inv_prime_prod, uint32_t *padding);

/* ---- ModUp (ModSwitch.cu:429-509), no terminal primes ----
 * src: L limbs (NTT domain). dst: beta blocks of (L+alpha) limbs,
 * beta = ceil(L/alpha). Returns beta. */
int orc_mod_up(uint32_t *dst, const uint32_t *src, int L,
               const uint32_t *q_primes, const uint32_t *p_primes, int alpha,
               int log_n);
/* ModUp of a level with prime_offset = max_ter - num_ter terminal primes
 * missing in front: group g covers the level's limbs
 * [max(0, g alpha - off), min((g+1) alpha, L + off) - off); empty groups
 * (ending at or before off) are left untouched. Returns beta =
 * ceil((L + off) / alpha), the number of group slots in dst. */
int orc_mod_up_ex(uint32_t *dst, const uint32_t *src, int L,
                  const uint32_t *q_primes, const uint32_t *p_primes,
                  int alpha, int prime_offset, int log_n);

/* ---- ModDown family (ModSwitch.cu:566-684), no terminal primes ----
 * src holds src_total limbs with primes src_primes; the first dst_len limbs
 * are kept, limbs [dst_len, src_total) are divided out.
 *   ModDown:           src_total = L+alpha, dst_len = L
 *   ModDownAndRescale: src_total = L+alpha, dst_len = L-k
 *   Rescale:           src_total = L,       dst_len = L-k            */
void orc_mod_down(uint32_t *dst, const uint32_t *src, int src_total,
                  const uint32_t *src_primes, int dst_len, int log_n);
/* The general ModDown with terminal primes and the BitPacker restore: source
 * limbs drop[0..num_drop) (indices into src) are divided out; destination
 * limb k (prime dst_primes[k]) keeps source limb dst_src[k], or is a
 * restored prime when dst_src[k] < 0 (its value is then -BConv / D).
 * The result is scaled by R = prod of the restored primes. */
void orc_mod_down_ex(uint32_t *dst, const uint32_t *src,
                     const uint32_t *src_primes, const int *drop, int num_drop,
                     const uint32_t *dst_primes, int dst_len,
                     const int *dst_src, int log_n);

/* ---- element-wise (ElementWise.cu:225-391, 504-575) ---- */
void orc_tensor(uint32_t *bx, uint32_t *ax, uint32_t *rx, const uint32_t *b1,
                const uint32_t *a1, const uint32_t *b2, const uint32_t *a2,
                int num_limbs, const uint32_t *primes, int log_n);
/* acc_{b,a}[l] = sum_g MontMul(modup[g][l], key_{b,a}[g][l']) over L+alpha
 * limbs; l' = l for l < L and max_q + (l - L) for aux limbs. */
void orc_paccum(uint32_t *acc_b, uint32_t *acc_a, const uint32_t *modup,
                int beta, const uint32_t *key_b, const uint32_t *key_a, int L,
                int alpha, int max_q, const uint32_t *primes, int log_n);
/* PAccum over the non-empty ModUp groups of a level with a prime offset:
 * modup group j pairs with key group key_group[j]; q limb l reads key limb
 * key_off + l, aux limb L + k reads max_q + k. */
void orc_paccum_ex(uint32_t *acc_b, uint32_t *acc_a, const uint32_t *modup,
                   int num_groups, const int *key_group, const uint32_t *key_b,
                   const uint32_t *key_a, int L, int alpha, int max_q,
                   int key_off, const uint32_t *primes, int log_n);
/* acc[l] += MontMul(p_prod[l], ct[l]) for l < L */
void orc_caccum(uint32_t *acc, const uint32_t *ct, const uint32_t *p_prod,
                int L, const uint32_t *primes, int log_n);
/* acc[l] = (acc[l] + MontMul(pt[l], x[l])) mod q_l over num_limbs limbs:
 * one term of the giant-step plaintext accumulation (GSFusedKernel,
 * Hoist.cu:80-118); threaded over limbs (orc_set_threads) */
void orc_pmult_accum(uint32_t *acc, const uint32_t *pt, const uint32_t *x,
                     int num_limbs, const uint32_t *primes, int log_n);
/* p_prod[l] = ToMont(prod(P) mod q_l) (Context.cpp:85-98) */
void orc_p_prod(uint32_t *p_prod, const uint32_t *q_primes, int L,
                const uint32_t *p_primes, int alpha);
/* NTT-domain automorphism X -> X^galois (ElementWise.cu:370-391) */
void orc_permute(uint32_t *dst, const uint32_t *src, int num_limbs, int log_n,
                 uint32_t galois);
uint32_t orc_galois_factor(int rot, int log_n);

/* ---- key-switch compositions (Context.cpp:584-871) ----
 * key_{b,a}: beta blocks of (max_q+alpha) limbs; q_primes has >= L entries.
 * hmult: res has L-1 limbs when rescale, L otherwise. */
int orc_hmult(uint32_t *res_b, uint32_t *res_a, const uint32_t *b1,
              const uint32_t *a1, const uint32_t *b2, const uint32_t *a2,
              const uint32_t *key_b, const uint32_t *key_a, int L, int max_q,
              const uint32_t *q_primes, const uint32_t *p_primes, int alpha,
              int log_n, int rescale);
int orc_rescale(uint32_t *res, const uint32_t *src, int L,
                const uint32_t *q_primes, int drop, int log_n);
/* MultKey on (b, a): returns (b + KS_b(a), KS_a(a)) with L limbs */
int orc_mult_key(uint32_t *res_b, uint32_t *res_a, const uint32_t *b,
                 const uint32_t *a, const uint32_t *key_b,
                 const uint32_t *key_a, int L, int max_q,
                 const uint32_t *q_primes, const uint32_t *p_primes, int alpha,
                 int log_n);
/* HRot = Permute(MultKey(ct), 5^rot mod 2N) (Context.cpp:776-791) */
int orc_hrot(uint32_t *res_b, uint32_t *res_a, const uint32_t *b,
             const uint32_t *a, const uint32_t *key_b, const uint32_t *key_a,
             int L, int max_q, const uint32_t *q_primes,
             const uint32_t *p_primes, int alpha, int log_n, int rot);

#ifdef __cplusplus
}
#endif

#endif
