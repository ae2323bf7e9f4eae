// Public C-ABI (include/cheddar_amd.h) over the C++ host classes, plus the
// error plumbing shared with the kernel-level ABI.
#include <climits>
#include <cstring>
#include <exception>
#include <memory>
#include <string>
#include <vector>

#include "cheddar.h"
#include "capi_internal.h"
#include "cheddar_amd.h"
#include "kernel_common.h"
#include "prime_math.h"

namespace {
thread_local std::string g_err;
}

namespace chd {
int set_error(int code, const std::string &msg) {
  g_err = msg;
  return code;
}
int check_launch(const char *where) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(CHD_ERR_HIP, std::string(where) + ": " +
                                      hipGetErrorString(e));
  return 0;
}
}  // namespace chd

using cheddar::Context;
using cheddar::Parameter;
using chd::set_error;
using chd_capi::LevelOk;
using chd_capi::MakeEvk;
using word = uint32_t;

struct chd_ntt_plan {
  std::unique_ptr<cheddar::ChainTables> chain;
};

struct chd_bconv_plan {
  std::unique_ptr<cheddar::ChainTables> dst_chain;
  std::vector<word> const1;
  std::vector<int32_t> const2;
  cheddar::DevBuf table;
  int src_len = 0, dst_len = 0;
};


extern "C" const char *chd_last_error(void) { return g_err.c_str(); }
extern "C" const char *chd_version(void) { return "cheddar-amd 0.1 gfx950"; }

// ------------------------------------------------------------ NTT plans --
extern "C" int chd_ntt_plan_create(chd_ntt_plan **out, int log_degree,
                                   const uint32_t *primes, int num_primes) {
  if (!out || !primes || num_primes < 1)
    return set_error(CHD_ERR_ARG, "chd_ntt_plan_create: invalid argument");
  CHD_TRY
  auto plan = std::make_unique<chd_ntt_plan>();
  plan->chain = std::make_unique<cheddar::ChainTables>(
      log_degree, std::vector<word>(primes, primes + num_primes));
  *out = plan.release();
  return 0;
  CHD_CATCH("chd_ntt_plan_create")
}

extern "C" void chd_ntt_plan_destroy(chd_ntt_plan *plan) { delete plan; }

extern "C" const void *chd_ntt_plan_tables(const chd_ntt_plan *plan) {
  return plan ? &plan->chain->tables() : nullptr;
}

static chd_limb_map PlainMap(int num_limbs) {
  chd_limb_map m{};
  m.num_q = num_limbs;
  m.skip_lo = INT_MAX;
  return m;
}

extern "C" int chd_ntt_forward(const chd_ntt_plan *plan, uint32_t *dst,
                               const uint32_t *src, int num_limbs,
                               int num_polys, int mont_conv, void *stream) {
  if (!plan || !dst || !src || num_limbs < 1 ||
      num_limbs > plan->chain->size() || num_polys < 1)
    return set_error(CHD_ERR_ARG, "chd_ntt_forward: invalid argument");
  chd_limb_map m = PlainMap(num_limbs);
  const long long ps = static_cast<long long>(num_limbs) << 16;
  return chd_k_ntt_fwd(&plan->chain->tables(), &m, dst, ps, src, ps,
                       num_limbs, num_polys,
                       mont_conv ? plan->chain->mont_converter() : nullptr,
                       stream);
}

extern "C" int chd_ntt_forward_two_pass(const chd_ntt_plan *plan,
                                        uint32_t *dst, const uint32_t *src,
                                        int num_limbs, int num_polys,
                                        int mont_conv, void *stream) {
  if (!plan || !dst || !src || num_limbs < 1 ||
      num_limbs > plan->chain->size() || num_polys < 1)
    return set_error(CHD_ERR_ARG,
                     "chd_ntt_forward_two_pass: invalid argument");
  chd_limb_map m = PlainMap(num_limbs);
  const long long ps = static_cast<long long>(num_limbs) << 16;
  return chd_k_ntt_fwd_2p(&plan->chain->tables(), &m, dst, ps, src, ps,
                          num_limbs, num_polys,
                          mont_conv ? plan->chain->mont_converter() : nullptr,
                          stream);
}

extern "C" int chd_ntt_inverse(const chd_ntt_plan *plan, uint32_t *dst,
                               const uint32_t *src, int num_limbs,
                               int num_polys, int mont_conv, void *stream) {
  if (!plan || !dst || !src || num_limbs < 1 ||
      num_limbs > plan->chain->size() || num_polys < 1)
    return set_error(CHD_ERR_ARG, "chd_ntt_inverse: invalid argument");
  chd_limb_map m = PlainMap(num_limbs);
  const long long ps = static_cast<long long>(num_limbs) << 16;
  return chd_k_ntt_inv(&plan->chain->tables(), &m, dst, ps, src, ps,
                       num_limbs, num_polys,
                       mont_conv ? plan->chain->inv_degree()
                                 : plan->chain->inv_degree_mont(),
                       0, stream);
}

extern "C" int chd_ntt_inverse_single_pass(const chd_ntt_plan *plan,
                                           uint32_t *dst, const uint32_t *src,
                                           int num_limbs, int num_polys,
                                           int mont_conv, void *stream) {
  if (!plan || !dst || !src || num_limbs < 1 ||
      num_limbs > plan->chain->size() || num_polys < 1)
    return set_error(CHD_ERR_ARG,
                     "chd_ntt_inverse_single_pass: invalid argument");
  chd_limb_map m = PlainMap(num_limbs);
  const long long ps = static_cast<long long>(num_limbs) << 16;
  return chd_k_ntt_inv_1p(&plan->chain->tables(), &m, dst, ps, src, ps,
                          num_limbs, num_polys,
                          mont_conv ? plan->chain->inv_degree()
                                    : plan->chain->inv_degree_mont(),
                          0, stream);
}

// ---------------------------------------------------------- BConv plans --
extern "C" int chd_bconv_plan_create(chd_bconv_plan **out, int log_degree,
                                     const uint32_t *src_primes, int src_len,
                                     const uint32_t *dst_primes,
                                     int dst_len) {
  if (!out || !src_primes || !dst_primes || src_len < 1 || src_len > 32 ||
      dst_len < 1)
    return set_error(CHD_ERR_ARG, "chd_bconv_plan_create: invalid argument");
  CHD_TRY
  namespace pm = cheddar::pm;
  auto plan = std::make_unique<chd_bconv_plan>();
  std::vector<word> src(src_primes, src_primes + src_len);
  std::vector<word> dst(dst_primes, dst_primes + dst_len);
  plan->dst_chain = std::make_unique<cheddar::ChainTables>(log_degree, dst);
  plan->src_len = src_len;
  plan->dst_len = dst_len;
  pm::modswitch_constants(src, dst, 1u << log_degree, 0, 0, &plan->const1,
                          &plan->const2);
  std::vector<unsigned char> packed(
      static_cast<size_t>(chd_bconv_table_size(src_len, dst_len)));
  int st = chd_bconv_table_pack(packed.data(), plan->const2.data(), dst.data(),
                                src_len, dst_len);
  if (st != 0) return st;
  plan->table.Resize(packed.size());
  plan->table.Upload(packed.data(), packed.size());
  *out = plan.release();
  return 0;
  CHD_CATCH("chd_bconv_plan_create")
}

extern "C" void chd_bconv_plan_destroy(chd_bconv_plan *plan) { delete plan; }

extern "C" int chd_bconv_plan_constants(const chd_bconv_plan *plan,
                                        uint32_t *const1, int32_t *const2) {
  if (!plan) return set_error(CHD_ERR_ARG, "chd_bconv_plan_constants");
  if (const1)
    std::memcpy(const1, plan->const1.data(), plan->const1.size() * 4);
  if (const2)
    std::memcpy(const2, plan->const2.data(), plan->const2.size() * 4);
  return 0;
}

extern "C" int chd_bconv_apply(const chd_bconv_plan *plan, uint32_t *dst,
                               const int32_t *src, void *stream) {
  if (!plan || !dst || !src)
    return set_error(CHD_ERR_ARG, "chd_bconv_apply: invalid argument");
  chd_limb_map m = PlainMap(plan->dst_len);
  return chd_k_bconv(&plan->dst_chain->tables(), &m, dst, src, plan->src_len,
                     plan->dst_len, plan->table.as<void>(), stream);
}

// ---------------------------------------------------- Parameter/Context --
extern "C" int chd_param_create(chd_param **out, int log_degree,
                                double base_scale,
                                int default_encryption_level,
                                const int *level_config, int num_levels,
                                const uint32_t *main_primes, int num_main,
                                const uint32_t *aux_primes, int num_aux,
                                const uint32_t *ter_primes, int num_ter) {
  if (!out || !level_config || num_levels < 1 || !main_primes ||
      num_main < 1 || !aux_primes || num_aux < 1 || num_ter < 0 ||
      (num_ter > 0 && !ter_primes))
    return set_error(CHD_ERR_ARG, "chd_param_create: invalid argument");
  CHD_TRY
  std::vector<std::pair<int, int>> lc;
  for (int i = 0; i < num_levels; i++)
    lc.emplace_back(level_config[2 * i], level_config[2 * i + 1]);
  auto p = std::make_unique<chd_param>();
  p->p = std::make_unique<Parameter<word>>(
      log_degree, base_scale, default_encryption_level, lc,
      std::vector<word>(main_primes, main_primes + num_main),
      std::vector<word>(aux_primes, aux_primes + num_aux),
      std::vector<word>(ter_primes, ter_primes + num_ter));
  *out = p.release();
  return 0;
  CHD_CATCH("chd_param_create")
}

extern "C" int chd_param_create_json(chd_param **out, const char *json_text) {
  if (!out || !json_text)
    return set_error(CHD_ERR_ARG, "chd_param_create_json: invalid argument");
  CHD_TRY
  auto p = std::make_unique<chd_param>();
  p->p = cheddar::ParameterFromJson(json_text);
  *out = p.release();
  return 0;
  CHD_CATCH("chd_param_create_json")
}

extern "C" void chd_param_destroy(chd_param *param) { delete param; }

extern "C" int chd_param_num_q(const chd_param *param, int level) {
  if (!param || level < 0 || level > param->p->max_level_) return -1;
  return param->p->LevelToNP(level).GetNumQ();
}

extern "C" int chd_param_alpha(const chd_param *param) {
  return param ? param->p->alpha_ : -1;
}

extern "C" int chd_param_max_level(const chd_param *param) {
  return param ? param->p->max_level_ : -1;
}

extern "C" int chd_param_evk_limbs(const chd_param *param) {
  if (!param) return -1;
  return param->p->GetMaxNumMain() + param->p->GetMaxNumTer() +
         param->p->alpha_;
}

extern "C" int chd_context_create(chd_context **out, const chd_param *param) {
  if (!out || !param)
    return set_error(CHD_ERR_ARG, "chd_context_create: invalid argument");
  CHD_TRY
  auto c = std::make_unique<chd_context>();
  c->c = Context<word>::Create(*param->p);
  *out = c.release();
  return 0;
  CHD_CATCH("chd_context_create")
}

extern "C" void chd_context_destroy(chd_context *ctx) { delete ctx; }

extern "C" int chd_context_beta(const chd_context *ctx, int level) {
  if (!ctx || level < 0 || level > ctx->c->param_.max_level_) return -1;
  return ctx->c->mod_switch_handlers_.at(level).GetBeta();
}

extern "C" int chd_tensor(const chd_context *ctx, int level, uint32_t *res_bx,
                          uint32_t *res_ax, uint32_t *res_rx,
                          const uint32_t *a_bx, const uint32_t *a_ax,
                          const uint32_t *b_bx, const uint32_t *b_ax,
                          void *stream) {
  CHD_CALL("chd_tensor",
           LevelOk(ctx, level) && res_bx && res_ax && res_rx && a_bx && a_ax &&
               b_bx && b_ax,
           ctx->c->TensorV(level, {res_bx, res_ax, res_rx}, {a_bx, a_ax, nullptr},
                           {b_bx, b_ax, nullptr}))
}

extern "C" int chd_mod_up(const chd_context *ctx, int level,
                          uint32_t *const *dst, const uint32_t *src,
                          void *stream) {
  CHD_CALL("chd_mod_up", LevelOk(ctx, level) && dst && src, {
    const auto &p = ctx->c->param_;
    const int n = p.degree_, nq = p.LevelToNP(level).GetNumQ();
    const auto &ms = ctx->c->mod_switch_handlers_.at(level);
    std::vector<cheddar::DvView<word>> v;
    for (int g = 0; g < ms.GetBeta(); g++) {
      // groups before FirstGroup() hold no limb of this level: unused
      if (!dst[g] && g >= ms.FirstGroup())
        throw cheddar::Error("null ModUp destination");
      v.emplace_back(dst[g], (nq + p.alpha_) * n, p.alpha_ * n);
    }
    ms.ModUp(v, cheddar::DvConstView<word>(src, nq * n, 0));
  })
}

extern "C" int chd_mod_down(const chd_context *ctx, int level, uint32_t *dst,
                            const uint32_t *src, void *stream) {
  CHD_CALL("chd_mod_down", LevelOk(ctx, level) && dst && src, {
    const auto &p = ctx->c->param_;
    const int n = p.degree_, nq = p.LevelToNP(level).GetNumQ();
    cheddar::DvView<word> d(dst, nq * n, 0);
    ctx->c->mod_switch_handlers_.at(level).ModDown(
        d, cheddar::DvConstView<word>(src, (nq + p.alpha_) * n, p.alpha_ * n));
  })
}

extern "C" int chd_rescale_poly(const chd_context *ctx, int level,
                                uint32_t *dst, const uint32_t *src,
                                void *stream) {
  CHD_CALL("chd_rescale_poly", LevelOk(ctx, level) && level > 0 && dst && src, {
    const auto &p = ctx->c->param_;
    const int n = p.degree_, nq = p.LevelToNP(level).GetNumQ();
    const int nq1 = p.LevelToNP(level - 1).GetNumQ();
    cheddar::DvView<word> d(dst, nq1 * n, 0);
    ctx->c->mod_switch_handlers_.at(level).Rescale(
        d, cheddar::DvConstView<word>(src, nq * n, 0));
  })
}

extern "C" int chd_mod_down_and_rescale(const chd_context *ctx, int level,
                                        uint32_t *dst, const uint32_t *src,
                                        void *stream) {
  CHD_CALL("chd_mod_down_and_rescale",
           LevelOk(ctx, level) && level > 0 && dst && src, {
             const auto &p = ctx->c->param_;
             const int n = p.degree_, nq = p.LevelToNP(level).GetNumQ();
             const int nq1 = p.LevelToNP(level - 1).GetNumQ();
             cheddar::DvView<word> d(dst, nq1 * n, 0);
             ctx->c->mod_switch_handlers_.at(level).ModDownAndRescale(
                 d, cheddar::DvConstView<word>(src, (nq + p.alpha_) * n,
                                               p.alpha_ * n));
           })
}

extern "C" int chd_hmult(const chd_context *ctx, int level, uint32_t *res_bx,
                         uint32_t *res_ax, const uint32_t *a_bx,
                         const uint32_t *a_ax, const uint32_t *b_bx,
                         const uint32_t *b_ax, const uint32_t *const *evk_bx,
                         const uint32_t *const *evk_ax, int evk_beta,
                         int rescale, void *stream) {
  CHD_CALL("chd_hmult",
           LevelOk(ctx, level) && (!rescale || level > 0) && res_bx &&
               res_ax && a_bx && a_ax && b_bx && b_ax && evk_bx && evk_ax &&
               evk_beta > 0,
           ctx->c->HMultV(level, {res_bx, res_ax, nullptr},
                          {a_bx, a_ax, nullptr}, {b_bx, b_ax, nullptr},
                          MakeEvk(ctx, evk_bx, evk_ax, evk_beta),
                          rescale != 0))
}

extern "C" int chd_rescale(const chd_context *ctx, int level, uint32_t *res_bx,
                           uint32_t *res_ax, const uint32_t *a_bx,
                           const uint32_t *a_ax, void *stream) {
  CHD_CALL("chd_rescale",
           LevelOk(ctx, level) && level > 0 && res_bx && res_ax && a_bx &&
               a_ax && res_bx != a_bx && res_ax != a_ax,
           ctx->c->RescaleV(level, {res_bx, res_ax, nullptr},
                            {a_bx, a_ax, nullptr}))
}

extern "C" int chd_mult_key(const chd_context *ctx, int level,
                            uint32_t *res_bx, uint32_t *res_ax,
                            const uint32_t *a_bx, const uint32_t *a_ax,
                            const uint32_t *const *evk_bx,
                            const uint32_t *const *evk_ax, int evk_beta,
                            void *stream) {
  CHD_CALL("chd_mult_key",
           LevelOk(ctx, level) && res_bx && res_ax && a_bx && a_ax && evk_bx &&
               evk_ax && evk_beta > 0,
           ctx->c->MultKeyV(level, {res_bx, res_ax, nullptr},
                            {a_bx, a_ax, nullptr},
                            MakeEvk(ctx, evk_bx, evk_ax, evk_beta)))
}

namespace {
// [a, a + aw) and [b, b + bw) (words) share memory
bool Overlap(const void *a, size_t aw, const void *b, size_t bw) {
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(a);
  const uintptr_t b0 = reinterpret_cast<uintptr_t>(b);
  return a0 < b0 + 4 * bw && b0 < a0 + 4 * aw;
}
}  // namespace

extern "C" int chd_mult_key_no_mod_down(const chd_context *ctx, int level,
                                        uint32_t *acc_b, uint32_t *acc_a,
                                        const uint32_t *a_bx,
                                        const uint32_t *a_ax,
                                        const uint32_t *a_rx,
                                        const uint32_t *const *evk_bx,
                                        const uint32_t *const *evk_ax,
                                        int evk_beta, void *stream) {
  CHD_CALL("chd_mult_key_no_mod_down",
           LevelOk(ctx, level) && acc_b && acc_a && a_bx && a_ax && evk_bx &&
               evk_ax && evk_beta > 0,
           {
             const auto &p = ctx->c->param_;
             const size_t qw =
                 static_cast<size_t>(p.LevelToNP(level).GetNumQ()) * p.degree_;
             const size_t tw = qw + static_cast<size_t>(p.alpha_) * p.degree_;
             // Context.cpp:657-658: no in-place operation
             bool bad = Overlap(acc_b, tw, acc_a, tw);
             for (const uint32_t *in : {a_bx, a_ax, a_rx})
               bad = bad || (in != nullptr && (Overlap(acc_b, tw, in, qw) ||
                                               Overlap(acc_a, tw, in, qw)));
             if (bad)
               throw cheddar::Error(
                   "In-place operation is not supported for "
                   "MultKeyNoModDown (the accumulator overlaps an input)");
             const auto key = MakeEvk(ctx, evk_bx, evk_ax, evk_beta);
             if (a_rx != nullptr)
               ctx->c->KeyMultNoModDownV(level, acc_b, acc_a, a_rx, a_bx, a_ax,
                                         key);
             else
               ctx->c->KeyMultNoModDownV(level, acc_b, acc_a, a_ax, a_bx,
                                         nullptr, key);
           })
}

extern "C" int chd_mult_key_no_mod_down_mod_up(
    const chd_context *ctx, int level, uint32_t *acc_b, uint32_t *acc_a,
    const uint32_t *const *a_modup, const uint32_t *const *evk_bx,
    const uint32_t *const *evk_ax, int evk_beta, void *stream) {
  CHD_CALL("chd_mult_key_no_mod_down_mod_up",
           LevelOk(ctx, level) && acc_b && acc_a && a_modup && evk_bx &&
               evk_ax && evk_beta > 0,
           {
             const auto &p = ctx->c->param_;
             const size_t tw =
                 static_cast<size_t>(p.LevelToNP(level).GetNumQ() + p.alpha_) *
                 p.degree_;
             const auto &ms = ctx->c->mod_switch_handlers_.at(level);
             bool bad = Overlap(acc_b, tw, acc_a, tw);
             for (int g = ms.FirstGroup(); g < ms.GetBeta(); g++)
               bad = bad || (a_modup[g] != nullptr &&
                             (Overlap(acc_b, tw, a_modup[g], tw) ||
                              Overlap(acc_a, tw, a_modup[g], tw)));
             if (bad)
               throw cheddar::Error(
                   "MultKeyNoModDown: the accumulator overlaps a ModUp group");
             ctx->c->KeyMultModUpV(level, acc_b, acc_a, a_modup,
                                   MakeEvk(ctx, evk_bx, evk_ax, evk_beta));
           })
}

extern "C" int chd_hrot(const chd_context *ctx, int level, uint32_t *res_bx,
                        uint32_t *res_ax, const uint32_t *a_bx,
                        const uint32_t *a_ax, const uint32_t *const *evk_bx,
                        const uint32_t *const *evk_ax, int evk_beta, int rot,
                        int num_slots, void *stream) {
  CHD_CALL("chd_hrot",
           LevelOk(ctx, level) && res_bx && res_ax && a_bx && a_ax &&
               res_bx != a_bx && res_ax != a_ax && evk_bx && evk_ax &&
               evk_beta > 0 && num_slots > 0,
           {
             int r = rot % num_slots;
             if (r < 0) r += num_slots;
             if (r == 0) throw cheddar::Error("HRot by 0 is not a rotation");
             const auto &p = ctx->c->param_;
             const size_t words =
                 static_cast<size_t>(p.LevelToNP(level).GetNumQ()) * p.degree_;
             cheddar::Workspace::Use use_ws(ctx->c->GetWorkspace());
             cheddar::Scratch t(ctx->c->GetWorkspace(), 2 * words);
             ctx->c->MultKeyV(level, {t.data(), t.data() + words, nullptr},
                              {a_bx, a_ax, nullptr},
                              MakeEvk(ctx, evk_bx, evk_ax, evk_beta));
             ctx->c->PermuteV(level, {res_bx, res_ax, nullptr},
                              {t.data(), t.data() + words, nullptr}, r);
           })
}

extern "C" int chd_permute(const chd_context *ctx, int level, uint32_t *res_bx,
                           uint32_t *res_ax, const uint32_t *a_bx,
                           const uint32_t *a_ax, int rot, void *stream) {
  CHD_CALL("chd_permute",
           LevelOk(ctx, level) && res_bx && res_ax && a_bx && a_ax &&
               res_bx != a_bx && res_ax != a_ax,
           ctx->c->PermuteV(level, {res_bx, res_ax, nullptr},
                            {a_bx, a_ax, nullptr}, rot))
}

namespace {
// ciphertext copy of two device polynomials of `limbs` limbs (the C-ABI's
// inputs are raw pointers; the hoisting engine works on Ciphertext objects)
cheddar::Ciphertext<word> CtCopy(const cheddar::Parameter<word> &p, int level,
                                 const uint32_t *bx, const uint32_t *ax) {
  cheddar::Ciphertext<word> ct(p.LevelToNP(level));
  const size_t bytes = ct.bx_.size() * sizeof(word);
  cheddar::HipCheck(hipMemcpyAsync(ct.bx_.data(), bx, bytes,
                                   hipMemcpyDeviceToDevice,
                                   cheddar::CurrentStream()),
                    "hipMemcpyAsync");
  cheddar::HipCheck(hipMemcpyAsync(ct.ax_.data(), ax, bytes,
                                   hipMemcpyDeviceToDevice,
                                   cheddar::CurrentStream()),
                    "hipMemcpyAsync");
  return ct;
}

cheddar::HoistHandler<word>::KeyLookup Keys(const chd_context *ctx,
                                            int num_keys, const int *key_rot,
                                            const uint32_t *const *key_bx,
                                            const uint32_t *const *key_ax,
                                            int key_beta) {
  return [=](int r) {
    for (int i = 0; i < num_keys; i++)
      if (key_rot[i] == r)
        return MakeEvk(ctx, key_bx + static_cast<size_t>(i) * key_beta,
                       key_ax + static_cast<size_t>(i) * key_beta, key_beta);
    throw cheddar::Error("no rotation key for " + std::to_string(r));
  };
}
}  // namespace

extern "C" int chd_hoist_baby_steps(
    const chd_context *ctx, int level, const uint32_t *ct_bx,
    const uint32_t *ct_ax, int num_rot, const int *rots,
    uint32_t *const *dst_bx, uint32_t *const *dst_ax, int num_keys,
    const int *key_rot, const uint32_t *const *key_bx,
    const uint32_t *const *key_ax, int key_beta, void *stream) {
  CHD_CALL("chd_hoist_baby_steps",
           LevelOk(ctx, level) && ct_bx && ct_ax && num_rot > 0 && rots &&
               dst_bx && dst_ax && num_keys >= 0 && key_beta > 0 &&
               (num_keys == 0 || (key_rot && key_bx && key_ax)),
           {
             const auto &p = ctx->c->param_;
             // one plaintext slot per baby step makes the handler's index set
             cheddar::HoistHandler<word>::PtMap pts;
             for (int i = 0; i < num_rot; i++)
               pts[0].try_emplace(rots[i],
                                  p.LevelToNP(level, p.alpha_), p.degree_);
             cheddar::HoistHandler<word> h(ctx->c, std::move(pts), level, 1.0);
             const cheddar::Ciphertext<word> in = CtCopy(p, level, ct_bx, ct_ax);
             std::map<int, cheddar::Ciphertext<word>> bs;
             h.BabyStep(*ctx->c, bs, in,
                        Keys(ctx, num_keys, key_rot, key_bx, key_ax, key_beta));
             for (int i = 0; i < num_rot; i++) {
               const auto &ct = bs.at(rots[i]);
               const size_t bytes = ct.bx_.size() * sizeof(word);
               if (!dst_bx[i] || !dst_ax[i])
                 throw cheddar::Error("null baby-step destination");
               cheddar::HipCheck(
                   hipMemcpyAsync(dst_bx[i], ct.bx_.data(), bytes,
                                  hipMemcpyDeviceToDevice,
                                  cheddar::CurrentStream()),
                   "hipMemcpyAsync");
               cheddar::HipCheck(
                   hipMemcpyAsync(dst_ax[i], ct.ax_.data(), bytes,
                                  hipMemcpyDeviceToDevice,
                                  cheddar::CurrentStream()),
                   "hipMemcpyAsync");
             }
             // the temporaries are freed on return: finish the copies first
             cheddar::HipCheck(hipStreamSynchronize(cheddar::CurrentStream()),
                               "hipStreamSynchronize");
           })
}

struct chd_hoist {
  std::shared_ptr<cheddar::Context<word>> c;
  std::unique_ptr<cheddar::HoistHandler<word>> own;
  std::unique_ptr<cheddar::LinearTransform<word>> lt;
  const cheddar::HoistHandler<word> *h = nullptr;  // own's or lt's
  int level;
  // buffers kept across runs: the input copy, the baby steps, the result
  cheddar::Ciphertext<word> in, res;
  std::map<int, cheddar::Ciphertext<word>> babies;
};

extern "C" int chd_hoist_create(chd_hoist **out, const chd_context *ctx,
                                int level, int num_gs, const int *gs,
                                int num_bs, const int *bs,
                                const uint32_t *const *pt, void *stream) {
  if (!out || !LevelOk(ctx, level) || level < 1 || num_gs < 1 || !gs ||
      num_bs < 1 || !bs || !pt)
    return set_error(CHD_ERR_ARG, "chd_hoist_create: invalid argument");
  CHD_TRY cheddar::StreamScope scope(static_cast<hipStream_t>(stream));
  const auto &p = ctx->c->param_;
  const cheddar::NPInfo np = p.LevelToNP(level, p.alpha_);
  cheddar::HoistHandler<word>::PtMap pts;
  for (int g = 0; g < num_gs; g++)
    for (int b = 0; b < num_bs; b++) {
      const uint32_t *src = pt[static_cast<size_t>(g) * num_bs + b];
      if (src == nullptr) continue;
      auto &pl = pts[gs[g]].try_emplace(bs[b], np, p.degree_).first->second;
      cheddar::HipCheck(hipMemcpyAsync(pl.mx_.data(), src,
                                       pl.mx_.size() * sizeof(word),
                                       hipMemcpyDeviceToDevice,
                                       cheddar::CurrentStream()),
                        "hipMemcpyAsync");
    }
  std::unique_ptr<chd_hoist> h(new chd_hoist);
  h->c = ctx->c;
  h->level = level;
  h->own.reset(new cheddar::HoistHandler<word>(ctx->c, std::move(pts), level,
                                               1.0));
  h->h = h->own.get();
  cheddar::HipCheck(hipStreamSynchronize(cheddar::CurrentStream()),
                    "hipStreamSynchronize");
  *out = h.release();
  return 0;
  CHD_CATCH("chd_hoist_create")
}

extern "C" int chd_hoist_create_from_messages(
    chd_hoist **out, const chd_context *ctx, int level, double pt_scale,
    int num_gs, const int *gs, int num_bs, const int *bs,
    const double *const *msg_re, const double *const *msg_im,
    const int *msg_len, int suppress_bs_swap, void *stream) {
  if (!out || !LevelOk(ctx, level) || level < 1 || num_gs < 1 || !gs ||
      num_bs < 1 || !bs || !msg_re || !msg_im || !msg_len)
    return set_error(CHD_ERR_ARG,
                     "chd_hoist_create_from_messages: invalid argument");
  CHD_TRY cheddar::StreamScope scope(static_cast<hipStream_t>(stream));
  cheddar::HoistHandler<word>::PlainHoistMap map;
  for (int g = 0; g < num_gs; g++)
    for (int b = 0; b < num_bs; b++) {
      const size_t k = static_cast<size_t>(g) * num_bs + b;
      if (msg_re[k] == nullptr) continue;
      if (msg_im[k] == nullptr || msg_len[k] < 1 ||
          msg_len[k] > ctx->c->param_.degree_ / 2)
        throw cheddar::Error("invalid message");
      cheddar::HoistHandler<word>::Message m(msg_len[k]);
      for (int i = 0; i < msg_len[k]; i++)
        m[i] = cheddar::Complex(msg_re[k][i], msg_im[k][i]);
      map[gs[g]][bs[b]] = std::move(m);
    }
  std::unique_ptr<chd_hoist> h(new chd_hoist);
  h->c = ctx->c;
  h->level = level;
  h->own.reset(new cheddar::HoistHandler<word>(ctx->c, map, level, pt_scale,
                                               suppress_bs_swap != 0));
  h->h = h->own.get();
  cheddar::HipCheck(hipStreamSynchronize(cheddar::CurrentStream()),
                    "hipStreamSynchronize");
  *out = h.release();
  return 0;
  CHD_CATCH("chd_hoist_create_from_messages")
}

extern "C" void chd_hoist_destroy(chd_hoist *h) { delete h; }

namespace {
int HoistRun(const char *name, const chd_hoist *h, uint32_t *res_bx,
             uint32_t *res_ax, const uint32_t *ct_bx, const uint32_t *ct_ax,
             int num_keys, const int *key_rot, const uint32_t *const *key_bx,
             const uint32_t *const *key_ax, int key_beta, bool min_ks,
             void *stream) {
  if (!h || !res_bx || !res_ax || !ct_bx || !ct_ax || num_keys < 0 ||
      key_beta < 1 || (num_keys > 0 && (!key_rot || !key_bx || !key_ax)))
    return set_error(CHD_ERR_ARG, std::string(name) + ": invalid argument");
  CHD_TRY cheddar::StreamScope scope(static_cast<hipStream_t>(stream));
  const auto &p = h->c->param_;
  chd_context view{h->c};
  const auto keys = Keys(&view, num_keys, key_rot, key_bx, key_ax, key_beta);
  chd_hoist *m = const_cast<chd_hoist *>(h);  // buffers, not the handler
  if (!(m->in.GetNP() == p.LevelToNP(h->level)) || m->in.bx_.size() == 0)
    m->in = cheddar::Ciphertext<word>(p.LevelToNP(h->level));
  const size_t in_bytes = m->in.bx_.size() * sizeof(word);
  cheddar::HipCheck(hipMemcpyAsync(m->in.bx_.data(), ct_bx, in_bytes,
                                   hipMemcpyDeviceToDevice,
                                   cheddar::CurrentStream()),
                    "hipMemcpyAsync");
  cheddar::HipCheck(hipMemcpyAsync(m->in.ax_.data(), ct_ax, in_bytes,
                                   hipMemcpyDeviceToDevice,
                                   cheddar::CurrentStream()),
                    "hipMemcpyAsync");
  h->h->BabyStep(*h->c, m->babies, m->in, keys, min_ks);
  h->h->GiantStep(*h->c, m->res, m->babies, keys, min_ks);
  const size_t bytes = m->res.bx_.size() * sizeof(word);
  cheddar::HipCheck(hipMemcpyAsync(res_bx, m->res.bx_.data(), bytes,
                                   hipMemcpyDeviceToDevice,
                                   cheddar::CurrentStream()),
                    "hipMemcpyAsync");
  cheddar::HipCheck(hipMemcpyAsync(res_ax, m->res.ax_.data(), bytes,
                                   hipMemcpyDeviceToDevice,
                                   cheddar::CurrentStream()),
                    "hipMemcpyAsync");
  return chd::check_launch(name);
  }
  catch (const std::exception &e) {
    return set_error(CHD_ERR_STATE, std::string(name) + ": " + e.what());
  }
}
}  // namespace

extern "C" int chd_hoist_run(const chd_hoist *h, uint32_t *res_bx,
                             uint32_t *res_ax, const uint32_t *ct_bx,
                             const uint32_t *ct_ax, int num_keys,
                             const int *key_rot, const uint32_t *const *key_bx,
                             const uint32_t *const *key_ax, int key_beta,
                             void *stream) {
  return HoistRun("chd_hoist_run", h, res_bx, res_ax, ct_bx, ct_ax, num_keys,
                  key_rot, key_bx, key_ax, key_beta, false, stream);
}

extern "C" int chd_hoist_run_min_ks(const chd_hoist *h, uint32_t *res_bx,
                                    uint32_t *res_ax, const uint32_t *ct_bx,
                                    const uint32_t *ct_ax, int num_keys,
                                    const int *key_rot,
                                    const uint32_t *const *key_bx,
                                    const uint32_t *const *key_ax,
                                    int key_beta, void *stream) {
  return HoistRun("chd_hoist_run_min_ks", h, res_bx, res_ax, ct_bx, ct_ax,
                  num_keys, key_rot, key_bx, key_ax, key_beta, true, stream);
}

extern "C" int chd_hoist_required_rotations(const chd_hoist *h, int min_ks,
                                            int *out, int capacity) {
  if (!h || capacity < 0 || (capacity > 0 && !out))
    return set_error(CHD_ERR_ARG,
                     "chd_hoist_required_rotations: invalid argument");
  CHD_TRY
  const std::set<int> r = h->h->RequiredRotations(min_ks != 0);
  int i = 0;
  for (int v : r) {
    if (i >= capacity) break;
    out[i++] = v;
  }
  return static_cast<int>(r.size());
  CHD_CATCH("chd_hoist_required_rotations")
}

extern "C" int chd_linear_transform_create(
    chd_hoist **out, const chd_context *ctx, int level, double pt_scale,
    int dim, int num_diag, const int *diag_idx, const double *const *diag_re,
    const double *const *diag_im, int bs, int gs, int pre_rotation,
    int additional_pt_rot, void *stream) {
  if (!out || !LevelOk(ctx, level) || level < 1 || dim < 1 ||
      dim > ctx->c->param_.degree_ / 2 || num_diag < 1 || !diag_idx ||
      !diag_re || !diag_im || bs < 1 || gs < 1)
    return set_error(CHD_ERR_ARG,
                     "chd_linear_transform_create: invalid argument");
  CHD_TRY cheddar::StreamScope scope(static_cast<hipStream_t>(stream));
  cheddar::StripedMatrix mat(dim, dim);
  for (int k = 0; k < num_diag; k++) {
    if (!diag_re[k] || !diag_im[k])
      throw cheddar::Error("null diagonal pointer");
    std::vector<cheddar::Complex> d(dim);
    for (int j = 0; j < dim; j++)
      d[j] = cheddar::Complex(diag_re[k][j], diag_im[k][j]);
    mat[diag_idx[k]] = std::move(d);
  }
  std::unique_ptr<chd_hoist> h(new chd_hoist);
  h->c = ctx->c;
  h->level = level;
  h->lt.reset(new cheddar::LinearTransform<word>(
      ctx->c, mat, level, pt_scale, bs, gs, pre_rotation, additional_pt_rot));
  h->h = &h->lt->GetHoistHandler();
  cheddar::HipCheck(hipStreamSynchronize(cheddar::CurrentStream()),
                    "hipStreamSynchronize");
  *out = h.release();
  return 0;
  CHD_CATCH("chd_linear_transform_create")
}



extern "C" int chd_hoist_evaluate(
    const chd_context *ctx, int level, uint32_t *res_bx, uint32_t *res_ax,
    const uint32_t *ct_bx, const uint32_t *ct_ax, int num_gs, const int *gs,
    int num_bs, const int *bs, const uint32_t *const *pt, int num_keys,
    const int *key_rot, const uint32_t *const *key_bx,
    const uint32_t *const *key_ax, int key_beta, void *stream) {
  CHD_CALL("chd_hoist_evaluate",
           LevelOk(ctx, level) && level > 0 && res_bx && res_ax && ct_bx &&
               ct_ax && num_gs > 0 && gs && num_bs > 0 && bs && pt &&
               num_keys >= 0 && key_beta > 0 &&
               (num_keys == 0 || (key_rot && key_bx && key_ax)),
           {
             const auto &p = ctx->c->param_;
             const cheddar::NPInfo np = p.LevelToNP(level, p.alpha_);
             cheddar::HoistHandler<word>::PtMap pts;
             for (int g = 0; g < num_gs; g++)
               for (int b = 0; b < num_bs; b++) {
                 const uint32_t *src = pt[static_cast<size_t>(g) * num_bs + b];
                 if (src == nullptr) continue;
                 auto &pl = pts[gs[g]].try_emplace(bs[b], np, p.degree_)
                                .first->second;
                 cheddar::HipCheck(
                     hipMemcpyAsync(pl.mx_.data(), src,
                                    pl.mx_.size() * sizeof(word),
                                    hipMemcpyDeviceToDevice,
                                    cheddar::CurrentStream()),
                     "hipMemcpyAsync");
               }
             cheddar::HoistHandler<word> h(ctx->c, std::move(pts), level, 1.0);
             const cheddar::Ciphertext<word> in = CtCopy(p, level, ct_bx, ct_ax);
             const auto keys =
                 Keys(ctx, num_keys, key_rot, key_bx, key_ax, key_beta);
             std::map<int, cheddar::Ciphertext<word>> babies;
             h.BabyStep(*ctx->c, babies, in, keys);
             cheddar::Ciphertext<word> res;
             h.GiantStep(*ctx->c, res, babies, keys);
             const size_t bytes = res.bx_.size() * sizeof(word);
             cheddar::HipCheck(hipMemcpyAsync(res_bx, res.bx_.data(), bytes,
                                              hipMemcpyDeviceToDevice,
                                              cheddar::CurrentStream()),
                               "hipMemcpyAsync");
             cheddar::HipCheck(hipMemcpyAsync(res_ax, res.ax_.data(), bytes,
                                              hipMemcpyDeviceToDevice,
                                              cheddar::CurrentStream()),
                               "hipMemcpyAsync");
             cheddar::HipCheck(hipStreamSynchronize(cheddar::CurrentStream()),
                               "hipStreamSynchronize");
           })
}

// --------------------------------------------------------- element-wise --
extern "C" int chd_elementwise(const chd_context *ctx, int level, int num_aux,
                               int op, int num_poly, uint32_t *const *dst,
                               const uint32_t *const *a,
                               const uint32_t *const *b, const uint32_t *cst,
                               void *stream) {
  CHD_CALL("chd_elementwise",
           LevelOk(ctx, level) && num_aux >= 0 &&
               num_aux <= ctx->c->param_.alpha_ && num_poly >= 1 &&
               num_poly <= CHD_MAX_POLY && dst && a && op >= CHD_EW_ADD &&
               op <= CHD_EW_COPY,
           {
             const auto &p = ctx->c->param_;
             const auto &eh = ctx->c->elem_handler_;
             const cheddar::NPInfo np = p.LevelToNP(level, num_aux);
             const int words = np.GetNumTotal() * p.degree_;
             const int aux = num_aux * p.degree_;
             std::vector<cheddar::DvView<word>> d;
             std::vector<cheddar::DvConstView<word>> x, y;
             for (int i = 0; i < num_poly; i++) {
               if (!dst[i] || !a[i]) throw cheddar::Error("null polynomial");
               d.emplace_back(dst[i], words, aux);
               x.emplace_back(a[i], words, aux);
             }
             const bool two = op == CHD_EW_ADD || op == CHD_EW_SUB ||
                              op == CHD_EW_MULT;
             if (two) {
               if (!b) throw cheddar::Error("missing second operand");
               for (int i = 0; i < num_poly; i++) {
                 if (!b[i]) throw cheddar::Error("null polynomial");
                 y.emplace_back(b[i], words, aux);
               }
             }
             const bool konst = op >= CHD_EW_ADD_CONST &&
                                op <= CHD_EW_MULT_CONST;
             if (konst && !cst) throw cheddar::Error("missing constant");
             const cheddar::DvConstView<word> c(cst, np.GetNumTotal(),
                                                num_aux);
             switch (op) {
               case CHD_EW_ADD: eh.Add(d, np, x, y); break;
               case CHD_EW_SUB: eh.Sub(d, np, x, y); break;
               case CHD_EW_NEG: eh.Neg(d, np, x); break;
               case CHD_EW_MULT: eh.Mult(d, np, x, y); break;
               case CHD_EW_PMULT:
                 if (!b || !b[0]) throw cheddar::Error("missing plaintext");
                 eh.PMult(d, np, x,
                          cheddar::DvConstView<word>(b[0], words, aux));
                 break;
               case CHD_EW_ADD_CONST: eh.AddConst(d, np, x, c); break;
               case CHD_EW_SUB_CONST: eh.SubConst(d, np, x, c); break;
               case CHD_EW_SUB_OPP_CONST:
                 eh.SubOppositeConst(d, np, x, c);
                 break;
               case CHD_EW_MULT_CONST: eh.MultConst(d, np, x, c); break;
               case CHD_EW_MULT_I: eh.MultImaginaryUnit(d, np, x); break;
               default: eh.Copy(d, np, x); break;
             }
           })
}

// ------------------------------------------------------------- encoder --
namespace {
std::vector<cheddar::Complex> Message(const double *re, const double *im,
                                      int len) {
  std::vector<cheddar::Complex> m(len);
  for (int i = 0; i < len; i++) m[i] = cheddar::Complex(re[i], im[i]);
  return m;
}
bool AuxOk(const Parameter<word> &p, int num_aux) {
  return num_aux == 0 || num_aux == p.alpha_;
}
int PaddedSlots(int len) {
  int s = 1;
  while (s < len) s <<= 1;
  return s;
}
}  // namespace

extern "C" int chd_encode(const chd_context *ctx, int level, int num_aux,
                          double scale, const double *msg_re,
                          const double *msg_im, int msg_len, uint32_t *dst,
                          void *stream) {
  if (!LevelOk(ctx, level) || !AuxOk(ctx->c->param_, num_aux) || !msg_re ||
      !msg_im || msg_len < 1 || msg_len > ctx->c->param_.degree_ / 2 || !dst)
    return set_error(CHD_ERR_ARG, "chd_encode: invalid argument");
  CHD_TRY cheddar::StreamScope scope(static_cast<hipStream_t>(stream));
  cheddar::Plaintext<word> pt;
  ctx->c->encoder_.Encode(pt, level, scale, Message(msg_re, msg_im, msg_len),
                          num_aux);
  cheddar::HipCheck(hipMemcpyAsync(dst, pt.mx_.data(),
                                   pt.mx_.size() * sizeof(word),
                                   hipMemcpyDeviceToDevice,
                                   cheddar::CurrentStream()),
                    "hipMemcpyAsync");
  cheddar::HipCheck(hipStreamSynchronize(cheddar::CurrentStream()),
                    "hipStreamSynchronize");
  return pt.GetNumSlots();
  CHD_CATCH("chd_encode")
}

extern "C" int chd_encode_constant(const chd_context *ctx, int level,
                                   int num_aux, double scale, double number,
                                   uint32_t *dst, void *stream) {
  CHD_CALL("chd_encode_constant",
           LevelOk(ctx, level) && AuxOk(ctx->c->param_, num_aux) && dst, {
             cheddar::Constant<word> c;
             ctx->c->encoder_.EncodeConstant(c, level, scale, number, num_aux);
             cheddar::HipCheck(hipMemcpyAsync(dst, c.cx_.data(),
                                              c.cx_.size() * sizeof(word),
                                              hipMemcpyDeviceToDevice,
                                              cheddar::CurrentStream()),
                               "hipMemcpyAsync");
             cheddar::HipCheck(
                 hipStreamSynchronize(cheddar::CurrentStream()),
                 "hipStreamSynchronize");
           })
}

extern "C" int chd_decode(const chd_context *ctx, int level, double scale,
                          int num_slots, const uint32_t *src, double *out_re,
                          double *out_im, void *stream) {
  CHD_CALL("chd_decode",
           LevelOk(ctx, level) && src && out_re && out_im && num_slots >= 1 &&
               num_slots <= ctx->c->param_.degree_ / 2 &&
               PaddedSlots(num_slots) == num_slots,
           {
             const auto &p = ctx->c->param_;
             cheddar::Plaintext<word> pt(p.LevelToNP(level), p.degree_);
             cheddar::HipCheck(hipMemcpyAsync(pt.mx_.data(), src,
                                              pt.mx_.size() * sizeof(word),
                                              hipMemcpyDeviceToDevice,
                                              cheddar::CurrentStream()),
                               "hipMemcpyAsync");
             pt.SetNumSlots(num_slots);
             pt.SetScale(scale);
             std::vector<cheddar::Complex> m;
             ctx->c->encoder_.Decode(m, pt);
             for (int i = 0; i < num_slots; i++) {
               out_re[i] = m[i].real();
               out_im[i] = m[i].imag();
             }
           })
}

extern "C" int chd_encode_coefficients(const chd_param *param, int level,
                                       int num_aux, double scale,
                                       const double *msg_re,
                                       const double *msg_im, int msg_len,
                                       uint32_t *host_out) {
  if (!param || level < 0 || level > param->p->max_level_ ||
      !AuxOk(*param->p, num_aux) || !msg_re || !msg_im || msg_len < 1 ||
      msg_len > param->p->degree_ / 2 || !host_out)
    return set_error(CHD_ERR_ARG, "chd_encode_coefficients: invalid argument");
  CHD_TRY
  const cheddar::Encoder<word> enc(*param->p);
  const int slots = PaddedSlots(msg_len);
  std::vector<cheddar::Complex> m = Message(msg_re, msg_im, msg_len);
  m.resize(slots);
  const std::vector<word> r =
      enc.CoefficientResidues(level, scale, std::move(m), num_aux);
  std::memcpy(host_out, r.data(), r.size() * sizeof(word));
  return slots;
  CHD_CATCH("chd_encode_coefficients")
}
