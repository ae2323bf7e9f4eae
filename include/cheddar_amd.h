/*
 * Public C-ABI of the MI355X-native CKKS key-switch path.
 *
 * This is the drop-in boundary a foreign caller binds (ctypes / cgo / JNI):
 * plain pointers and sizes, device pointers for ciphertext data, an explicit
 * stream (hipStream_t passed as void*, NULL = the null stream, which is the
 * reference's only stream). The functions wrap the C++ classes of
 * cheddar-fhe_amd/host (cheddar::Parameter, Context, ...), which keep the
 * reference's C++ API (include/core/Parameter.h:42-47, Context.h:70-423).
 *
 * Conventions (identical to the reference):
 *  - u32 residues, primes q < 2^31, q = 1 mod 2N, N = 2^16;
 *  - limb-major polynomials u32[limbs][N], limb order ter (reversed), main,
 *    aux (include/core/Parameter.h:198-206);
 *  - ciphertext and key data in the NTT domain, Montgomery form (x 2^32);
 *  - an evaluation key is beta pairs (bx_g, ax_g), each of
 *    (max main + max ter + alpha) limbs (include/core/Container.h:289-345).
 * Every call returns CHD_OK (0) or a negative status; chd_last_error()
 * returns the message of the last failure on the calling thread. No call
 * exits the process (the reference's AssertTrue -> exit(1) becomes a status).
 * Calls that overlap on one stream are ordered by it; a Context is not
 * thread-safe (as in the reference).
 */
#ifndef CHEDDAR_AMD_H
#define CHEDDAR_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CHD_OK 0
#define CHD_ERR_INVALID_ARGUMENT (-1)
#define CHD_ERR_HIP (-2)
#define CHD_ERR_STATE (-3)
#define CHD_ERR_ALLOC (-4)

const char *chd_last_error(void);
const char *chd_version(void);

/* ---------------------------------------------------------------------- */
/* standalone NTT over an explicit prime chain (configs 1-2)               */
/* replaces NTTHandler::NTT / INTT (include/core/NTT.h:56-61)              */
/* ---------------------------------------------------------------------- */
typedef struct chd_ntt_plan chd_ntt_plan;
int chd_ntt_plan_create(chd_ntt_plan **out, int log_degree,
                        const uint32_t *primes, int num_primes);
void chd_ntt_plan_destroy(chd_ntt_plan *plan);
/* device tables of the plan (for the kernel-level ABI, cheddar_kernels.h) */
const void *chd_ntt_plan_tables(const chd_ntt_plan *plan);
/* [num_polys][num_limbs][N]; limb i uses prime i of the plan.
 * forward: natural -> bit-reversed, mont_conv multiplies by 2^32 first.
 * inverse: mont_conv=1 returns intt * 2^-32 (the reference's default),
 *          0 returns intt exactly. dst may equal src. */
int chd_ntt_forward(const chd_ntt_plan *plan, uint32_t *dst,
                    const uint32_t *src, int num_limbs, int num_polys,
                    int mont_conv, void *stream);
int chd_ntt_inverse(const chd_ntt_plan *plan, uint32_t *dst,
                    const uint32_t *src, int num_limbs, int num_polys,
                    int mont_conv, void *stream);
/* chd_ntt_forward on the two passes (chd_k_ntt_fwd_2p): the same results;
 * slower for one call at a time, faster in throughput when several streams
 * keep the GPU busy. No reference counterpart. */
int chd_ntt_forward_two_pass(const chd_ntt_plan *plan, uint32_t *dst,
                             const uint32_t *src, int num_limbs,
                             int num_polys, int mont_conv, void *stream);
/* chd_ntt_inverse on the single-pass kernel (chd_k_ntt_inv_1p): the same
 * results, one HBM read and write per limb; dst must not overlap src. For
 * comparison with the default two-pass inverse, which is faster at config 2.
 * No reference counterpart. */
int chd_ntt_inverse_single_pass(const chd_ntt_plan *plan, uint32_t *dst,
                                const uint32_t *src, int num_limbs,
                                int num_polys, int mont_conv, void *stream);

/* ---------------------------------------------------------------------- */
/* standalone BConv between explicit prime sets (config 3)                 */
/* replaces ModSwitchMatrixMult (src/core/ModSwitch.cu:23-171) with the    */
/* table of PopulateModSwitchConstants (ModSwitch.cu:320-370)              */
/* ---------------------------------------------------------------------- */
typedef struct chd_bconv_plan chd_bconv_plan;
int chd_bconv_plan_create(chd_bconv_plan **out, int log_degree,
                          const uint32_t *src_primes, int src_len,
                          const uint32_t *dst_primes, int dst_len);
void chd_bconv_plan_destroy(chd_bconv_plan *plan);
/* host copies of the reference-form constants: const1[src_len] =
 * (N prod_{j!=i} q_j)^-1 mod q_i, const2[dst_len][src_len] =
 * centre(qhat_i 2^64 mod p_k) */
int chd_bconv_plan_constants(const chd_bconv_plan *plan, uint32_t *const1,
                             int32_t *const2);
/* dst[k] = sum_i src[i] const2[k][i] 2^-32 mod p_k; src centred int32
 * [src_len][N], dst [dst_len][N] */
int chd_bconv_apply(const chd_bconv_plan *plan, uint32_t *dst,
                    const int32_t *src, void *stream);

/* ---------------------------------------------------------------------- */
/* Parameter / Context (include/core/Parameter.h:42-47, Context.h:70)      */
/* ---------------------------------------------------------------------- */
typedef struct chd_param chd_param;
typedef struct chd_context chd_context;

/* level_config: num_levels pairs (num_main, num_ter), as the JSON
 * "level_config"; ter_primes may be NULL when num_ter == 0. */
int chd_param_create(chd_param **out, int log_degree, double base_scale,
                     int default_encryption_level, const int *level_config,
                     int num_levels, const uint32_t *main_primes, int num_main,
                     const uint32_t *aux_primes, int num_aux,
                     const uint32_t *ter_primes, int num_ter);
/* A parameter set from the reference's JSON layout (the files in parameters/:
 * log_degree, log_default_scale, default_encryption_level, main_primes,
 * terminal_primes, auxiliary_primes, level_config, additional_base), the
 * file's text in json_text (unittest/Testbed.h:95-179). */
int chd_param_create_json(chd_param **out, const char *json_text);
void chd_param_destroy(chd_param *param);
/* number of q limbs (main + ter) at a level; -1 on error */
int chd_param_num_q(const chd_param *param, int level);
int chd_param_alpha(const chd_param *param);
int chd_param_max_level(const chd_param *param);
/* limb count of an evaluation key (max main + max ter + alpha) */
int chd_param_evk_limbs(const chd_param *param);

int chd_context_create(chd_context **out, const chd_param *param);
void chd_context_destroy(chd_context *ctx);
/* beta = number of dnum groups of ModUp at this level (ModSwitch.cu:181) */
int chd_context_beta(const chd_context *ctx, int level);

/* Polynomials below hold num_q(level) limbs unless stated; aux-extended
 * polynomials hold num_q(level) + alpha limbs. */

/* Context::Mult(Ct,Ct) -> Tensor (Context.cpp:316-330) */
int chd_tensor(const chd_context *ctx, int level, uint32_t *res_bx,
               uint32_t *res_ax, uint32_t *res_rx, const uint32_t *a_bx,
               const uint32_t *a_ax, const uint32_t *b_bx,
               const uint32_t *b_ax, void *stream);
/* ModSwitchHandler::ModUp (ModSwitch.cu:429-509): dst[beta] each
 * num_q + alpha limbs, beta = chd_context_beta(level). Dnum groups sit on
 * the chain's positions: at a level missing terminal primes the leading
 * groups that hold none of its limbs are not written (their pointers may be
 * NULL). */
int chd_mod_up(const chd_context *ctx, int level, uint32_t *const *dst,
               const uint32_t *src, void *stream);
/* ModDown: (num_q + alpha) -> num_q limbs (ModSwitch.cu:511-527) */
int chd_mod_down(const chd_context *ctx, int level, uint32_t *dst,
                 const uint32_t *src, void *stream);
/* Rescale: num_q -> num_q(level-1) limbs (ModSwitch.cu:529-545) */
int chd_rescale_poly(const chd_context *ctx, int level, uint32_t *dst,
                     const uint32_t *src, void *stream);
/* merged ModDownAndRescale: (num_q + alpha) -> num_q(level-1) limbs
 * (ModSwitch.cu:547-564) */
int chd_mod_down_and_rescale(const chd_context *ctx, int level, uint32_t *dst,
                             const uint32_t *src, void *stream);

/* HMult (Context.cpp:862-871): res = relinearize(a * b), rescaled when
 * rescale != 0 (res then has num_q(level-1) limbs). evk_bx/evk_ax: beta
 * device pointers, each chd_param_evk_limbs() limbs. res may alias a. */
int chd_hmult(const chd_context *ctx, int level, uint32_t *res_bx,
              uint32_t *res_ax, const uint32_t *a_bx, const uint32_t *a_ax,
              const uint32_t *b_bx, const uint32_t *b_ax,
              const uint32_t *const *evk_bx, const uint32_t *const *evk_ax,
              int evk_beta, int rescale, void *stream);
/* chd_hmult without allocation. No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same arguments,
 * kernels and results as chd_hmult; the key-switch temporaries come from a
 * static 64 MiB device array (one per GPU, held until the process ends)
 * instead of the context's arena, and the call makes no hipMalloc, hipFree
 * or other allocating call. A level whose HMult needs more than 64 MiB of
 * temporaries (more than 24 q limbs with alpha = 8, dnum 3) is rejected
 * with CHD_ERR_INVALID_ARGUMENT. Every call on one GPU shares that array,
 * and the library orders those calls itself: host threads take a
 * per-GPU lock, and a call on another stream than the previous call (of
 * any context) first makes its stream wait for that call's end, so calls
 * from several contexts and streams run one after another on the device
 * rather than at the same time. */
int chd_hmult_noalloc(const chd_context *ctx, int level, uint32_t *res_bx,
                      uint32_t *res_ax, const uint32_t *a_bx,
                      const uint32_t *a_ax, const uint32_t *b_bx,
                      const uint32_t *b_ax, const uint32_t *const *evk_bx,
                      const uint32_t *const *evk_ax, int evk_beta,
                      int rescale, void *stream);
/* Context::Rescale of a two-polynomial ciphertext (Context.cpp:739-774).
 * Both polynomials go through each phase together; the result may not
 * overlap the input (such a call fails, chd_last_error naming the
 * overlap). */
int chd_rescale(const chd_context *ctx, int level, uint32_t *res_bx,
                uint32_t *res_ax, const uint32_t *a_bx, const uint32_t *a_ax,
                void *stream);
/* Context::MultKey (Context.cpp:584-607): (b, a) -> (b + KS_b(a), KS_a(a)) */
int chd_mult_key(const chd_context *ctx, int level, uint32_t *res_bx,
                 uint32_t *res_ax, const uint32_t *a_bx, const uint32_t *a_ax,
                 const uint32_t *const *evk_bx, const uint32_t *const *evk_ax,
                 int evk_beta, void *stream);
/* Context::MultKeyNoModDown(accum, a, key) (Context.h:423,
 * Context.cpp:645-712): the key switch without its ModDown, for hoisting and
 * bootstrapping callers (Hoist.cu:676, 771, 849). acc_b / acc_a get
 * num_q(level) + alpha limbs: sum_g ModUp(d)_g * evk_g over the extended
 * basis, plus P * a_bx on the q limbs of acc_b, and P * a_ax on those of
 * acc_a when a_rx is given. d = a_rx when a_rx is not NULL
 * (relinearisation of a tensor), else a_ax (MultKey). The accumulators may
 * not overlap each other or an input (the reference's no-in-place rule). */
int chd_mult_key_no_mod_down(const chd_context *ctx, int level,
                             uint32_t *acc_b, uint32_t *acc_a,
                             const uint32_t *a_bx, const uint32_t *a_ax,
                             const uint32_t *a_rx,
                             const uint32_t *const *evk_bx,
                             const uint32_t *const *evk_ax, int evk_beta,
                             void *stream);
/* Context::MultKeyNoModDown(accum, a_modup, a_orig, key) (Context.h:421-422,
 * Context.cpp:609-643): the PAccum of a caller-held ModUp with the key,
 * a_modup[g] for g < chd_context_beta(level) as chd_mod_up writes it
 * (num_q + alpha limbs each; groups holding no limb of the level are not
 * read and may be NULL) -> acc_b / acc_a (num_q(level) + alpha limbs),
 * which may not overlap each other or a ModUp group. */
int chd_mult_key_no_mod_down_mod_up(const chd_context *ctx, int level,
                                    uint32_t *acc_b, uint32_t *acc_a,
                                    const uint32_t *const *a_modup,
                                    const uint32_t *const *evk_bx,
                                    const uint32_t *const *evk_ax,
                                    int evk_beta, void *stream);
/* Context::HRot (Context.cpp:776-791): MultKey then Permute by 5^rot;
 * num_slots as Ciphertext::GetNumSlots (N/2 for a fresh ciphertext).
 * res must not alias a. */
int chd_hrot(const chd_context *ctx, int level, uint32_t *res_bx,
             uint32_t *res_ax, const uint32_t *a_bx, const uint32_t *a_ax,
             const uint32_t *const *evk_bx, const uint32_t *const *evk_ax,
             int evk_beta, int rot, int num_slots, void *stream);
/* Permute of a ciphertext by 5^rot (rot = -1: conjugation), no key switch
 * (Context.cpp:501-527) */
int chd_permute(const chd_context *ctx, int level, uint32_t *res_bx,
                uint32_t *res_ax, const uint32_t *a_bx, const uint32_t *a_ax,
                int rot, void *stream);

/* ---------------------------------------------------------------------- */
/* Hoisted rotations (src/extension/Hoist.cu; include/extension/Hoist.h)   */
/* ---------------------------------------------------------------------- */
/* Rotation keys are passed as num_keys entries: key_rot[i] is the rotation
 * index, key_bx/key_ax[i * key_beta + g] its dnum group g (max-level limbs,
 * as for chd_hrot). Both calls synchronise the stream before returning.
 *
 * HoistHandler::EvaluateBabyStep (Hoist.cu:578-691), hoisted path: for
 * rotation rots[i] (0 <= r < N/2), (dst_bx[i], dst_ax[i]) gets the baby step
 * in the extended basis (num_q(level) + alpha limbs, not divided by P):
 * Permute(KeySwitchNoModDown(ct.ax) + PseudoModUp(ct.bx), r); r = 0 gives
 * (PseudoModUp(bx), PseudoModUp(ax)) with zero aux limbs. */
int chd_hoist_baby_steps(const chd_context *ctx, int level,
                         const uint32_t *ct_bx, const uint32_t *ct_ax,
                         int num_rot, const int *rots, uint32_t *const *dst_bx,
                         uint32_t *const *dst_ax, int num_keys,
                         const int *key_rot, const uint32_t *const *key_bx,
                         const uint32_t *const *key_ax, int key_beta,
                         void *stream);
/* A HoistHandler kept across calls (Hoist.h: the handler is built once
 * from its plaintexts, then evaluated many times): chd_hoist_create copies
 * the plaintexts (layout as for chd_hoist_evaluate) and synchronises the
 * stream; chd_hoist_run evaluates one ciphertext at the handler's level,
 * reusing the handler's baby-step and result buffers (no allocation after
 * the first run; runs of one handler must not overlap). */
typedef struct chd_hoist chd_hoist;
int chd_hoist_create(chd_hoist **out, const chd_context *ctx, int level,
                     int num_gs, const int *gs, int num_bs, const int *bs,
                     const uint32_t *const *pt, void *stream);
/* The reference's message constructor (Hoist.cu:131-177): messages
 * msg_re / msg_im [g * num_bs + b] of msg_len[g * num_bs + b] complex values
 * (NULL when absent) are encoded at (level, alpha aux primes) with pt_scale;
 * a map with the single giant step 0 is evaluated with baby and giant steps
 * swapped (messages rotated right by their baby step) unless
 * suppress_bs_swap is non-zero. Synchronises the stream. */
int chd_hoist_create_from_messages(chd_hoist **out, const chd_context *ctx,
                                   int level, double pt_scale, int num_gs,
                                   const int *gs, int num_bs, const int *bs,
                                   const double *const *msg_re,
                                   const double *const *msg_im,
                                   const int *msg_len, int suppress_bs_swap,
                                   void *stream);
void chd_hoist_destroy(chd_hoist *h);
int chd_hoist_run(const chd_hoist *h, uint32_t *res_bx, uint32_t *res_ax,
                  const uint32_t *ct_bx, const uint32_t *ct_ax, int num_keys,
                  const int *key_rot, const uint32_t *const *key_bx,
                  const uint32_t *const *key_ax, int key_beta, void *stream);
/* HoistHandler::Evaluate with min_ks (Hoist.cu:517-566): baby steps by
 * repeated HRot with the baby-step stride, giant steps Horner-style with the
 * giant-step stride, then Rescale; only the two stride keys are needed.
 * Same arguments as chd_hoist_run. */
int chd_hoist_run_min_ks(const chd_hoist *h, uint32_t *res_bx,
                         uint32_t *res_ax, const uint32_t *ct_bx,
                         const uint32_t *ct_ax, int num_keys,
                         const int *key_rot, const uint32_t *const *key_bx,
                         const uint32_t *const *key_ax, int key_beta,
                         void *stream);
/* HoistHandler::AddRequiredRotations (Hoist.cu:978-1004): writes up to
 * capacity rotation indices (ascending) into out and returns how many the
 * handler needs. */
int chd_hoist_required_rotations(const chd_hoist *h, int min_ks, int *out,
                                 int capacity);
/* LinearTransform (src/extension/LinearTransform.cpp:40-88): a dim x dim
 * matrix (dim a power of two) given by num_diag generalised diagonals,
 * diagonal diag_idx[k] = (diag_re[k][j], diag_im[k][j]) = M[j][(j + i) % dim],
 * as a hoisting handle (run with chd_hoist_run / chd_hoist_run_min_ks,
 * destroy with chd_hoist_destroy). bs, gs, pre_rotation and
 * additional_pt_rot have the reference's meaning. Synchronises the stream. */
int chd_linear_transform_create(chd_hoist **out, const chd_context *ctx,
                                int level, double pt_scale, int dim,
                                int num_diag, const int *diag_idx,
                                const double *const *diag_re,
                                const double *const *diag_im, int bs, int gs,
                                int pre_rotation, int additional_pt_rot,
                                void *stream);
/* HoistHandler::Evaluate (Hoist.cu:569-576, 840-975, 487-515): baby steps
 * bs[0..num_bs), giant steps gs[0..num_gs) (gs must contain 0 when
 * num_gs > 1), plaintexts pt[g * num_bs + b] (num_q(level) + alpha limbs in
 * the NTT domain, Montgomery form, or NULL when absent);
 * res (num_q(level - 1) limbs) = ModDownAndRescale(
 *     sum_g Rot_g(sum_b pt[g][b] * Rot_b(ct))) with double hoisting. */
int chd_hoist_evaluate(const chd_context *ctx, int level, uint32_t *res_bx,
                       uint32_t *res_ax, const uint32_t *ct_bx,
                       const uint32_t *ct_ax, int num_gs, const int *gs,
                       int num_bs, const int *bs, const uint32_t *const *pt,
                       int num_keys, const int *key_rot,
                       const uint32_t *const *key_bx,
                       const uint32_t *const *key_ax, int key_beta,
                       void *stream);

/* ElementWiseHandler ops (src/core/ElementWise.cu:687-920, 1673-1706) on
 * num_poly (1..3) polynomials of num_q(level) + num_aux limbs, canonical in
 * and out: op is one of CHD_EW_* (include/cheddar_kernels.h); b[p] is read
 * by ADD / SUB / MULT, b[0] by PMULT (one plaintext for every polynomial);
 * cst (one Montgomery-form value per limb, a Constant's cx_) by the *_CONST
 * ops. dst may alias a or b. */
int chd_elementwise(const chd_context *ctx, int level, int num_aux, int op,
                    int num_poly, uint32_t *const *dst,
                    const uint32_t *const *a, const uint32_t *const *b,
                    const uint32_t *cst, void *stream);

/* ------------------------------------------------------------ encoder --
 * Encoder::Encode (src/core/Encode.cpp:23-43, 84-109, 135-190): the message
 * (msg_re[i], msg_im[i], i < msg_len, zero-padded to the next power of two
 * slots) -> dst (device, (num_q(level) + num_aux) * N words, the plaintext
 * in the NTT domain, Montgomery form). num_aux is 0 or alpha (a plaintext
 * for the extended basis, Hoist.cu:131-145). Returns the padded slot count
 * (> 0) or a negative error code. Synchronises the stream. */
int chd_encode(const chd_context *ctx, int level, int num_aux, double scale,
               const double *msg_re, const double *msg_im, int msg_len,
               uint32_t *dst, void *stream);
/* Encoder::EncodeConstant (Encode.cpp:248-273): trunc(number * scale) mod
 * each prime, Montgomery form, into dst (device, num_q(level) + num_aux
 * words). Synchronises the stream. */
int chd_encode_constant(const chd_context *ctx, int level, int num_aux,
                        double scale, double number, uint32_t *dst,
                        void *stream);
/* Encoder::Decode (Encode.cpp:45-82, 192-246): src (device, num_q(level)
 * limbs in the NTT domain, Montgomery form) with num_slots slots (a power of
 * two <= N/2) at scale -> out_re / out_im (host, num_slots each).
 * Synchronises the stream. */
int chd_decode(const chd_context *ctx, int level, double scale, int num_slots,
               const uint32_t *src, double *out_re, double *out_im,
               void *stream);
/* The host half of chd_encode alone (no device): the coefficient residues
 * ComplexVectorToPlaintext writes before the NTT, [num_q(level) +
 * num_aux][N] words into host_out. Returns the padded slot count. */
int chd_encode_coefficients(const chd_param *param, int level, int num_aux,
                            double scale, const double *msg_re,
                            const double *msg_im, int msg_len,
                            uint32_t *host_out);

#ifdef __cplusplus
}
#endif

#endif
