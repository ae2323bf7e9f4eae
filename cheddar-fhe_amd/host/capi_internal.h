// Internals of the public C-ABI shared by its source files: the opaque
// handle types, argument helpers and the call wrapper that turns C++
// exceptions into status codes (include/cheddar_amd.h conventions).
#pragma once

#include <memory>
#include <string>

#include "cheddar.h"
#include "cheddar_amd.h"
#include "kernel_common.h"

struct chd_param {
  std::unique_ptr<cheddar::Parameter<uint32_t>> p;
};

struct chd_context {
  std::shared_ptr<cheddar::Context<uint32_t>> c;
};

#define CHD_TRY try {
#define CHD_CATCH(name)                                                     \
  }                                                                         \
  catch (const std::exception &e) {                                         \
    return chd::set_error(CHD_ERR_STATE, std::string(name ": ") + e.what()); \
  }

namespace chd_capi {

inline bool LevelOk(const chd_context *ctx, int level) {
  return ctx && level >= 0 && level <= ctx->c->param_.max_level_;
}

// the reference's EvaluationKey view: beta device pointers per part, each
// of max main + max ter + alpha limbs
inline cheddar::Context<uint32_t>::EvkRef MakeEvk(const chd_context *ctx,
                                                  const uint32_t *const *bx,
                                                  const uint32_t *const *ax,
                                                  int beta) {
  const auto &p = ctx->c->param_;
  cheddar::Context<uint32_t>::EvkRef r;
  r.np = cheddar::NPInfo(p.GetMaxNumMain(), p.GetMaxNumTer(), p.alpha_);
  for (int g = 0; g < beta; g++) {
    if (!bx[g] || !ax[g]) throw cheddar::Error("null evaluation-key pointer");
    r.bx.push_back(bx[g]);
    r.ax.push_back(ax[g]);
  }
  return r;
}

}  // namespace chd_capi

// argument check, then the body on the caller's stream; exceptions and
// launch errors become status codes
#define CHD_CALL(name, cond, ...)                                           \
  if (!(cond))                                                              \
    return chd::set_error(CHD_ERR_ARG, name ": invalid argument");          \
  CHD_TRY cheddar::StreamScope scope(static_cast<hipStream_t>(stream));     \
  __VA_ARGS__;                                                              \
  return chd::check_launch(name);                                           \
  CHD_CATCH(name)
