// chd_hmult_noalloc: HMult whose key-switch temporaries live in a file-scope
// device array instead of memory the library allocates, for callers that
// cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc). It runs the same kernels as chd_hmult;
// only where their scratch operands point differs.
#include <mutex>
#include <vector>

#include "capi_internal.h"

namespace {
// 64 MiB: HMult at N = 2^16 with up to 24 q limbs, alpha = 8 and dnum 3
// takes at most 50.5 MiB (the top level of config 4). Each GPU the library
// runs on holds its own copy until the process ends.
constexpr size_t kScratchBytes = 64ull << 20;
constexpr size_t kScratchWords = kScratchBytes / sizeof(uint32_t);
}  // namespace

static __device__ __align__(256) uint32_t scratch[kScratchWords];

namespace {
std::mutex g_mu;
// per device: the address of that device's copy of `scratch` (the array's
// name is a host-side stand-in, never a device address)
std::vector<uint32_t *> g_scratch_ptr;

// looked up once per device, with that device current
int ScratchOfCurrentDevice(uint32_t **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return chd::set_error(CHD_ERR_HIP, std::string("chd_hmult_noalloc: "
                                                   "hipGetDevice: ") +
                                           hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_mu);
  if (dev >= static_cast<int>(g_scratch_ptr.size()))
    g_scratch_ptr.resize(dev + 1, nullptr);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return chd::set_error(CHD_ERR_HIP,
                            std::string("chd_hmult_noalloc: "
                                        "hipGetSymbolAddress: ") +
                                hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<uint32_t *>(p);
  }
  *out = g_scratch_ptr[dev];
  return 0;
}
}  // namespace

extern "C" int chd_hmult_noalloc(const chd_context *ctx, int level,
                                 uint32_t *res_bx, uint32_t *res_ax,
                                 const uint32_t *a_bx, const uint32_t *a_ax,
                                 const uint32_t *b_bx, const uint32_t *b_ax,
                                 const uint32_t *const *evk_bx,
                                 const uint32_t *const *evk_ax, int evk_beta,
                                 int rescale, void *stream) {
  using chd_capi::LevelOk;
  if (!(LevelOk(ctx, level) && (!rescale || level > 0) && res_bx && res_ax &&
        a_bx && a_ax && b_bx && b_ax && evk_bx && evk_ax && evk_beta > 0))
    return chd::set_error(CHD_ERR_ARG, "chd_hmult_noalloc: invalid argument");
  uint32_t *buf = nullptr;
  if (int st = ScratchOfCurrentDevice(&buf)) return st;
  CHD_TRY
  const size_t need = ctx->c->KeySwitchScratchWords(level, rescale != 0);
  if (need > kScratchWords)
    return chd::set_error(
        CHD_ERR_ARG,
        "chd_hmult_noalloc: this level needs " +
            std::to_string((need * sizeof(uint32_t) + (1 << 20) - 1) >> 20) +
            " MiB of scratch, more than the static " +
            std::to_string(kScratchBytes >> 20) + " MiB");
  cheddar::Workspace *ws = ctx->c->GetWorkspace();
  if (ws == nullptr)
    return chd::set_error(CHD_ERR_STATE, "chd_hmult_noalloc: no workspace");
  cheddar::StreamScope scope(static_cast<hipStream_t>(stream));
  cheddar::Workspace::Use use(ws);
  cheddar::Workspace::External ext(ws, buf, kScratchWords);
  ctx->c->HMultV(level, {res_bx, res_ax, nullptr}, {a_bx, a_ax, nullptr},
                 {b_bx, b_ax, nullptr},
                 chd_capi::MakeEvk(ctx, evk_bx, evk_ax, evk_beta),
                 rescale != 0);
  return chd::check_launch("chd_hmult_noalloc");
  CHD_CATCH("chd_hmult_noalloc")
}
