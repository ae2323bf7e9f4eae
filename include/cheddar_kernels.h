/*
 * Kernel-level C-ABI of the MI355X key-switch path: the thin layer between
 * the C++ handler classes (cheddar::NTTHandler, ModSwitchHandler,
 * ElementWiseHandler) and the hand-written gfx950 kernels. Plain C types,
 * raw device pointers, an explicit stream (hipStream_t passed as void*).
 * Every call returns 0 on success or a negative chd_status; the message is
 * available from chd_last_error() (declared in cheddar_amd.h).
 *
 * Each entry point replaces the CUDA launch sites named in its comment
 * (paths relative to the Cheddar reference tree). No entry point allocates
 * or frees device memory.
 */
#ifndef CHEDDAR_KERNELS_H
#define CHEDDAR_KERNELS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-prime device tables of one prime chain (ter reversed, main, aux).
 * Built by the C++ NTTHandler (src/core/NTT.cu:1233-1299 counterpart). */
typedef struct chd_tables {
  const uint32_t *q;        /* [T] primes                                 */
  const int32_t *qinv;      /* [T] q^-1 mod 2^32 (signed)                 */
  const uint32_t *tw;       /* [T][N] ToMont(psi^brev(j))                 */
  const uint32_t *itw;      /* [T][N] ToMont(psi^-brev(j))                */
  /* [T][4][N/4] ToMont(psi^-(s (2 brev_{log N - 2}(k) + 1))), s = 0..3: the
   * per-element twist of the single-pass inverse NTT's residue class s
   * (row 0 is ToMont(1)); optional: NULL keeps every inverse on the
   * two-pass kernels */
  const uint32_t *twist;
} chd_tables;

/* launch limb j -> logical limb l = j + (j >= skip_lo ? skip_len : 0);
 * aux limbs (l >= num_q) shift src/table/constant indices by their gaps
 * (the reference's PtrList extra_, include/common/PtrList.h:38-63). */
typedef struct chd_limb_map {
  int num_q;
  int skip_lo, skip_len;
  int src_gap;
  int tab_off, tab_gap;
  int cst_gap;
} chd_limb_map;

/* Forward NTT of num_limbs x num_polys limbs (NTT.cu:606-671, 815-887).
 * pre_cst != NULL: input first multiplied by MontMul(x, pre_cst[limb])
 * (Montgomery conversion). Strides are in words between polynomials. src
 * either is dst (in place: same stride and src_gap 0; two passes) or
 * overlaps none of dst's polynomials (one pass above 16 limbs, two up to
 * 16); any other overlap is rejected with CHD_ERR_INVALID_ARGUMENT before
 * a launch. */
int chd_k_ntt_fwd(const chd_tables *t, const chd_limb_map *m, uint32_t *dst,
                  long long dst_pstride, const uint32_t *src,
                  long long src_pstride, int num_limbs, int num_polys,
                  const uint32_t *pre_cst, void *stream);
/* The same transform, same arguments and overlap rules, always on the two
 * passes (no reference counterpart): slower than the single pass for one
 * call at a time (17.7 against 15.5 us at config 2), but its many short
 * workgroups share the GPU better with kernels of other streams (config-2
 * forward + inverse steps over two to four streams: 4-7 % more steps per
 * second), for callers that keep several streams busy. */
int chd_k_ntt_fwd_2p(const chd_tables *t, const chd_limb_map *m,
                     uint32_t *dst, long long dst_pstride,
                     const uint32_t *src, long long src_pstride,
                     int num_limbs, int num_polys, const uint32_t *pre_cst,
                     void *stream);

/* Forward NTT of dst in place followed by the ModDown epilogue
 * out = MontMul(MontMul(src2, pad) - NTT(x), inv_prod) (NTT.cu:889-971,
 * 456-601). src2 covers logical limbs [src2_lo, src2_hi); pad may be NULL. */
int chd_k_ntt_fwd_moddown(const chd_tables *t, const chd_limb_map *m,
                          uint32_t *dst, int num_limbs, const uint32_t *src2,
                          int src2_lo, int src2_hi, const uint32_t *inv_prod,
                          const uint32_t *pad, void *stream);

/* Same for num_polys (<= CHD_MAX_JOBS) polynomials in separate buffers dst[p];
 * src2 of polynomial p is at src2 + p * src2_pstride. With src == NULL the
 * NTT runs in place on dst[p]; otherwise its input is src + p * src_pstride,
 * which must not overlap any dst[p] (one HBM pass instead of two). */
int chd_k_ntt_fwd_moddown_multi(const chd_tables *t, const chd_limb_map *m,
                                uint32_t *const *dst, int num_polys,
                                int num_limbs, const uint32_t *src,
                                long long src_pstride, const uint32_t *src2,
                                long long src2_pstride, int src2_lo,
                                int src2_hi, const uint32_t *inv_prod,
                                const uint32_t *pad, void *stream);

/* The ModDown tail of a one-source switch (Rescale: ModSwitch.cu:529-545
 * through ModDownWorker 566-684) in one launch: for every limb l of
 * polynomial p, the one-source BConv (ModSwitch.cu:23-171 with src_len 1)
 * y_l = MontMul(src1_p, bconv1[l]) of the centred INTT output
 * src1_p = src1 + p * src1_pstride (one limb, signed), then the forward NTT
 * and the ModDown epilogue of chd_k_ntt_fwd_moddown_multi. y is never
 * stored. bconv1[l] is the BConv table entry of destination l, canonical.
 * No source or src2 limb may overlap a destination. */
int chd_k_ntt_fwd_moddown_bconv1_multi(
    const chd_tables *t, const chd_limb_map *m, uint32_t *const *dst,
    int num_polys, int num_limbs, const int32_t *src1, long long src1_pstride,
    const uint32_t *bconv1, const uint32_t *src2, long long src2_pstride,
    int src2_lo, int src2_hi, const uint32_t *inv_prod, const uint32_t *pad,
    void *stream);

/* Inverse NTT with epilogue MontMul(N*intt(x), cst[limb]), centred into
 * [-(q-1)/2, (q-1)/2] when centre (NTT.cu:673-813, 973-1128). src either
 * is dst (in place, same stride) or does not overlap it. */
int chd_k_ntt_inv(const chd_tables *t, const chd_limb_map *m, uint32_t *dst,
                  long long dst_pstride, const uint32_t *src,
                  long long src_pstride, int num_limbs, int num_polys,
                  const uint32_t *cst, int centre, void *stream);

/* chd_k_ntt_inv in one pass over residue classes of the output: workgroup
 * s of a limb reads the whole limb and writes its words 4u + s (one HBM read
 * and write per limb; the two passes read and write twice). src must not
 * overlap dst (else CHD_ERR_INVALID_ARGUMENT before any launch) and t->twist
 * must be set. Same results as chd_k_ntt_inv; slower at config 2 (21.5 us
 * against 19 us), kept for that comparison. No reference counterpart: an
 * alternative layout of INTT (NTT.cu:673-741). */
int chd_k_ntt_inv_1p(const chd_tables *t, const chd_limb_map *m,
                     uint32_t *dst, long long dst_pstride, const uint32_t *src,
                     long long src_pstride, int num_limbs, int num_polys,
                     const uint32_t *cst, int centre, void *stream);

/* Second pass of chd_k_ntt_inv alone (stages 7..0 and the epilogue, in
 * place on dst), for data whose first pass another kernel produced
 * (chd_keyacc_args intt_b / intt_a). */
int chd_k_ntt_inv_cols(const chd_tables *t, const chd_limb_map *m,
                       uint32_t *dst, long long dst_pstride, int num_limbs,
                       int num_polys, const uint32_t *cst, int centre,
                       void *stream);

/* chd_k_ntt_inv of the element-wise Montgomery product MontMul(src, src_mul)
 * (src_mul laid out like src). With src = a.ax, src_mul = b.ax this is the
 * Tensor's rx (ElementWise.cu:504-546) fed straight into ModUp's
 * INTTAndMultConst (ModSwitch.cu:442-447) without storing rx. */
int chd_k_ntt_inv_mul(const chd_tables *t, const chd_limb_map *m,
                      uint32_t *dst, long long dst_pstride,
                      const uint32_t *src, const uint32_t *src_mul,
                      long long src_pstride, int num_limbs, int num_polys,
                      const uint32_t *cst, int centre, void *stream);

/* BConv (src/core/ModSwitch.cu:23-171): for dst position k,
 * dst[pos(k)] = sum_i src[i] * T[k][i] * 2^-32 mod p_k with centred int32
 * sources, 1 <= src_len <= 32. table = chd_bconv_table_size(src_len,
 * dst_len) bytes made by chd_bconv_table_pack from the reference-form
 * table T (dst-major).
 * pos(k) = k + (k >= skip_lo ? skip_len : 0); prime of pos via m->tab_*.
 * chd_k_bconv writes its result with streaming stores (a standalone
 * conversion); chd_k_bconv_batch, the key switch's entry, with default
 * stores so that the next launch finds the result in the caches. */
long long chd_bconv_table_size(int src_len, int dst_len);
int chd_bconv_table_pack(void *host_out, const int32_t *table_ref,
                         const uint32_t *dst_primes, int src_len, int dst_len);
int chd_k_bconv(const chd_tables *t, const chd_limb_map *m, uint32_t *dst,
                const int32_t *src, int src_len, int dst_len,
                const void *table, void *stream);

/* Batched BConv: up to CHD_MAX_BCONV_JOBS independent conversions in one launch
 * (the beta groups of ModUp, or the two polynomials of ModDown). Each job
 * has its own source, table, lengths and skip range; all share the prime
 * mapping of m (dst positions are logical limbs of one level). */
#define CHD_MAX_JOBS 8
/* a BConv launch takes more jobs: every group of several ModUps */
#define CHD_MAX_BCONV_JOBS 32
typedef struct chd_bconv_job {
  uint32_t *dst;
  const int32_t *src;
  const void *table;
  int src_len, dst_len;
  int skip_lo, skip_len;
} chd_bconv_job;
int chd_k_bconv_batch(const chd_tables *t, const chd_limb_map *m,
                      const chd_bconv_job *jobs, int num_jobs, void *stream);

/* Column pass (stages 0..7) of NTTForModUp for all dnum groups in one launch:
 * group g's polynomial sits at modup + g * group_stride (group_limbs limbs,
 * in place) and its own limbs [max(0, g alpha - group_shift),
 * min((g+1) alpha - group_shift, m->num_q)) are skipped (NTT.cu:815-887;
 * group_shift as in chd_keyacc_args). with_rows also runs stages 8..15 (the
 * complete NTTForModUp); without it the data is left for
 * chd_k_modup_keyacc. */
int chd_k_ntt_fwd_groups(const chd_tables *t, const chd_limb_map *m,
                         uint32_t *modup, long long group_stride,
                         int num_groups, int alpha, int group_shift,
                         int group_limbs, int with_rows, void *stream);
/* The same for num_inputs (<= CHD_MAX_JOBS) ModUps of one level in one
 * launch: group g of input i at modup + (i * num_groups + g) * group_stride
 * (the batched giant steps of Hoist.cu:895-957). */
int chd_k_ntt_fwd_groups_batch(const chd_tables *t, const chd_limb_map *m,
                               uint32_t *modup, long long group_stride,
                               int num_groups, int num_inputs, int alpha,
                               int group_shift, int group_limbs,
                               int with_rows, void *stream);

/* Fused ModUp row pass + evaluation-key inner product + CAccum
 * (Context.cpp:609-712, ElementWise.cu:225-366):
 *   acc_{b,a}[l] = sum_g MontMul(u_g[l], key_g.{b,a}[l'])
 *                  + MontMul(p_prod[l], c{b,a}[l])   (q limbs only)
 * u_g[l] = d[l] on group g's own limbs, otherwise the forward NTT of the
 * column-pass data in modup (left by chd_k_ntt_fwd_groups). l' = l for q
 * limbs and l + key_gap/N for aux limbs. ca may be NULL (MultKey); cb NULL
 * skips the CAccum (a plain PAccum, MultKeyNoModDown of Context.cpp:609-643). */
typedef struct chd_keyacc_args {
  int num_q;
  int tab_off, tab_gap;
  /* beta non-empty ModUp groups; group g owns the level's limbs
   * [max(0, g alpha - group_shift), min((g+1) alpha - group_shift, num_q)),
   * group_shift = (max_ter - num_ter) mod alpha (ModSwitch.cu:440-470) */
  int alpha, beta, group_shift;
  const uint32_t *modup;
  long long group_stride;
  const uint32_t *d;
  const uint32_t *kb[CHD_MAX_JOBS];
  const uint32_t *ka[CHD_MAX_JOBS];
  long long key_gap;
  const uint32_t *p_prod;
  const uint32_t *cb;
  const uint32_t *ca;
  uint32_t *acc_b;
  uint32_t *acc_a;
  /* Tensor mode (HMult), selected by a1 != NULL: d, cb and ca are not read
   * but formed from the two input ciphertexts (b1, a1) x (b2, a2), q limbs
   * only, as Tensor computes them (ElementWise.cu:504-546):
   * d = rx = MontMul(a1, a2), cb = bx = MontMul(b1, b2),
   * ca = ax = MontMul(b1 - q + a1, b2 - q + a2) - bx - rx. */
  const uint32_t *b1, *a1, *b2, *a2;
  /* when set, added to acc_b on every limb (q and aux), unscaled: the
   * extended-basis b of a giant-step accumulator (Hoist.cu:940-957) */
  const uint32_t *add_b;
  /* when set (both), limbs l >= intt_lo of the accumulators are not stored:
   * the first pass of ModDown's INTT (stages 15..8, unreduced) goes to
   * intt_{b,a} + (l - intt_lo) N instead, for chd_k_ntt_inv_cols to finish */
  uint32_t *intt_b, *intt_a;
  int intt_lo;
} chd_keyacc_args;
int chd_k_modup_keyacc(const chd_tables *t, const chd_keyacc_args *args,
                       void *stream);
/* num_jobs (<= CHD_MAX_JOBS) independent key accumulations of one level
 * (same num_q and alpha; own inputs, keys and outputs each) in one launch. */
int chd_k_modup_keyacc_batch(const chd_tables *t, const chd_keyacc_args *jobs,
                             int num_jobs, void *stream);

/* Tensor (ElementWise.cu:504-575, 921-953): Karatsuba product of
 * (b1,a1) x (b2,a2) -> (bx, ax, rx) over num_limbs limbs. src2 == src1
 * selects the squaring kernel. src_gap as in chd_limb_map. */
int chd_k_tensor(const chd_tables *t, const chd_limb_map *m, uint32_t *bx,
                 uint32_t *ax, uint32_t *rx, const uint32_t *b1,
                 const uint32_t *a1, const uint32_t *b2, const uint32_t *a2,
                 int num_limbs, void *stream);

/* CPAccum / CPAccumAdd (ElementWise.cu:225-366, 1437-1643):
 * dst[p][i] = (src0[p][i]) + sum_a MontMul(common_a[., i], src_a[p][i]).
 * const_accum: common_a is one constant per limb; otherwise a polynomial. */
#define CHD_MAX_ACCUM 8
#define CHD_MAX_POLY 3
typedef struct chd_accum_src {
  const uint32_t *src[CHD_MAX_POLY];
  const uint32_t *common;
  long long src_gap;     /* words added to the index of aux limbs */
  long long common_gap;  /* same for common (limbs if const_accum) */
} chd_accum_src;
int chd_k_cpaccum(const chd_tables *t, const chd_limb_map *m,
                  uint32_t *const *dst, int num_polys, const uint32_t *const *src0,
                  long long src0_gap, const chd_accum_src *srcs, int num_accum,
                  int const_accum, int num_limbs, void *stream);

/* Permute (ElementWise.cu:370-391, 966-999): NTT-domain automorphism with
 * galois factor g: dst[l][x] = src[l][brev(((2 brev(x)+1) g - 1) mod 2N)]. */
int chd_k_permute(const chd_limb_map *m, uint32_t *const *dst,
                  const uint32_t *const *src, int num_polys, int num_limbs,
                  uint32_t galois, void *stream);

/* PermuteAccum / PermuteAccumAdd (ElementWise.cu:395-501, 1002-1110):
 * dst[p] = src0[p] (if given) + sum_j Permute(srcs[j].src[p], galois_j),
 * modular sums. Aux limbs of src0 / src_j are read src0_gap / src_gap words
 * further on. galois 1 adds a source unpermuted. dst may alias src0. */
typedef struct chd_perm_src {
  const uint32_t *src[CHD_MAX_POLY];
  uint32_t galois;
  long long src_gap;
} chd_perm_src;
int chd_k_permute_accum(const chd_tables *t, const chd_limb_map *m,
                        uint32_t *const *dst, int num_polys,
                        const uint32_t *const *src0, long long src0_gap,
                        const chd_perm_src *srcs, int num_src, int num_limbs,
                        void *stream);

/* Hoisted baby step, key multiply + automorphism fused (BSFusedKernel,
 * src/extension/Hoist.cu:20-78, 207-327). For every rotation k:
 *   t_b = sum_g u_g * key_k,g.b,  t_a = sum_g u_g * key_k,g.a  (q + alpha
 *   limbs), t_b += MontMul(ct_b, p_prod) on q limbs (PseudoModUp of b),
 *   dst_k = Permute((t_b, t_a), galois_k)
 * where u_g is dnum group g of ModUp(a): modup + g * group_stride, except on
 * the group's own limbs [g alpha, min((g+1) alpha, num_q)), where it is the
 * input limb d itself. Keys hold key_gap/N extra q limbs before their aux
 * limbs. Up to CHD_MAX_BS rotations and CHD_MAX_BS_GROUPS groups. */
/* dst[0..words) = 0 (words a multiple of 4, dst 16-byte aligned); a kernel,
 * not a memset node, so the call is safe inside captured graphs */
int chd_k_zero(uint32_t *dst, long long words, void *stream);

/* Hoisted giant-step plaintext accumulation (GSFusedKernel,
 * src/extension/Hoist.cu:80-118, 334-445): for every giant step g of the
 * launch, dst_g = [dst_g +] sum_b MontMul(pt[g][b], bs_b) for both parts,
 * over num_limbs extended-basis limbs. Each baby step is read once per
 * launch. pt[g][b] NULL skips the pair. */
#define CHD_GS_MAX_BS 32
#define CHD_GS_MAX_GS 8
typedef struct chd_gs_args {
  int num_bs, num_gs, add_to_dst;
  const uint32_t *bs_b[CHD_GS_MAX_BS], *bs_a[CHD_GS_MAX_BS];
  const uint32_t *pt[CHD_GS_MAX_GS][CHD_GS_MAX_BS];
  uint32_t *dst_b[CHD_GS_MAX_GS], *dst_a[CHD_GS_MAX_GS];
} chd_gs_args;
int chd_k_gs_fused(const chd_tables *t, const chd_limb_map *m,
                   const chd_gs_args *args, int num_limbs, void *stream);

/* The same for num_gs = 8, 16, 24, 28 or 32 giant steps in one launch, so
 * each baby step is read once for all of them. num_bs must be a multiple of
 * 4 (pad with zero baby steps). The plaintext addresses are a device array
 * pt_table[g * pt_stride + b]; every entry must be a valid plaintext (point
 * absent pairs at a zero plaintext). Inputs must be canonical residues.
 * pt_tiled (optional, NULL for none): the plaintexts of giant steps
 * g < tiled_rows in the tiled layout chd_k_gs_pack_tiled writes (rows =
 * tiled_rows); they are read from it instead of through pt_table, and the
 * giant steps from tiled_rows on (padding) are neither computed nor
 * written. */
#define CHD_GS_WIDE_GS 32
typedef struct chd_gs_wide_args {
  int num_bs, num_gs, add_to_dst, pt_stride;
  const uint32_t *bs_b[CHD_GS_MAX_BS], *bs_a[CHD_GS_MAX_BS];
  const uint32_t *const *pt_table;
  uint32_t *dst_b[CHD_GS_WIDE_GS], *dst_a[CHD_GS_WIDE_GS];
  const uint32_t *pt_tiled;
  int tiled_rows;
} chd_gs_wide_args;
int chd_k_gs_fused_wide(const chd_tables *t, const chd_limb_map *m,
                        const chd_gs_wide_args *args, int num_limbs,
                        void *stream);

/* Tiled copy of a giant-step plaintext table for chd_k_gs_fused_wide (no
 * counterpart in the reference, whose GSFusedKernel reads each plaintext of
 * its map in place, Hoist.cu:80-118): word c of 256-coefficient block k of
 * limb l of the plaintext pt_table[g * pt_stride + b] goes to
 *   dst[((((l * (N / 256) + k) * rows + g) * pt_stride + b) << 8) + c]
 * for g < rows, b < pt_stride, l < num_limbs, so the plaintexts one
 * accumulation workgroup reads (one block of one limb, every pair) are one
 * contiguous run. dst holds rows * pt_stride * num_limbs * N words. */
int chd_k_gs_pack_tiled(const uint32_t *const *pt_table, int rows,
                        int pt_stride, int num_limbs, uint32_t *dst,
                        void *stream);
/* The inverse for one row g of such a tiled array (rows x pt_stride
 * plaintexts of num_limbs limbs): the first dst_limbs limbs of plaintext
 * (g, b) go to dst + b * dst_limbs * N, for b < pt_stride (no counterpart in
 * the reference; it gives back the per-pair plaintexts of one giant step). */
int chd_k_gs_untile_row(const uint32_t *tiled, int rows, int pt_stride,
                        int num_limbs, int g, int dst_limbs, uint32_t *dst,
                        void *stream);

#define CHD_MAX_BS 8
#define CHD_MAX_BS_GROUPS 4
typedef struct chd_bs_args {
  /* groups as in chd_keyacc_args */
  int num_q, alpha, beta, group_shift, num_rot;
  const uint32_t *modup;
  long long group_stride;
  const uint32_t *d;
  const uint32_t *ct_b;
  const uint32_t *p_prod;
  const uint32_t *kb[CHD_MAX_BS][CHD_MAX_BS_GROUPS];
  const uint32_t *ka[CHD_MAX_BS][CHD_MAX_BS_GROUPS];
  long long key_gap;
  uint32_t galois[CHD_MAX_BS];
  uint32_t *dst_b[CHD_MAX_BS];
  uint32_t *dst_a[CHD_MAX_BS];
} chd_bs_args;
int chd_k_bs_fused(const chd_tables *t, const chd_limb_map *m,
                   const chd_bs_args *args, void *stream);

/* Element-wise ops over num_poly polynomials of m->num_q q limbs plus aux
 * limbs (ElementWise.cu:33-220, 600-660, Basic.cuh:169-260), canonical in
 * and out. b: per polynomial (ADD, SUB, MULT) or b[0] for every polynomial
 * (PMULT). cst: one value per limb (the *_CONST ops). MULT_I multiplies by
 * the imaginary unit X^(N/2), i.e. by +-ToMont(psi^(N/2)) of each limb (the
 * second entry of its twiddle table), negated in the upper half of the
 * evaluation points. a_gap / b_gap / cst_gap: aux-limb gaps as in
 * chd_limb_map.src_gap (in limbs, or entries for cst). */
#define CHD_EW_ADD 0
#define CHD_EW_SUB 1
#define CHD_EW_NEG 2
#define CHD_EW_MULT 3
#define CHD_EW_PMULT 4
#define CHD_EW_ADD_CONST 5
#define CHD_EW_SUB_CONST 6
#define CHD_EW_SUB_OPP_CONST 7
#define CHD_EW_MULT_CONST 8
#define CHD_EW_MULT_I 9
#define CHD_EW_COPY 10
typedef struct chd_ew_args {
  int op;
  int num_poly;
  uint32_t *dst[CHD_MAX_POLY];
  const uint32_t *a[CHD_MAX_POLY];
  const uint32_t *b[CHD_MAX_POLY];
  int a_gap, b_gap;
  const uint32_t *cst;
  int cst_gap;
} chd_ew_args;
int chd_k_elementwise(const chd_tables *t, const chd_limb_map *m,
                      const chd_ew_args *args, int num_limbs, void *stream);

#ifdef __cplusplus
}
#endif

#endif
