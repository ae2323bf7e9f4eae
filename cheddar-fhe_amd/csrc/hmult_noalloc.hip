// chd_hmult_noalloc: HMult whose key-switch temporaries live in a file-scope
// device array instead of memory the library allocates, for callers that
// cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc). It runs the same kernels as chd_hmult;
// only where their scratch operands point differs.
#include <memory>
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
// Per device: the address of that device's copy of `scratch` (the array's
// name is a host-side stand-in, never a device address), and what orders
// the calls that share it. Every context, stream and host thread of the
// process shares one device's array, so its calls are serialised on the
// host by `mu` and on the device by `done`: a call on another stream than
// the previous call first makes its stream wait for that call's end.
struct DeviceScratch {
  uint32_t *ptr = nullptr;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
  bool has_last = false;
  std::mutex mu;
};
std::mutex g_mu;
std::vector<std::unique_ptr<DeviceScratch>> g_scratch;

// set up once per device, with that device current: the array's address
// and the ordering event (no device memory is allocated)
int ScratchOfCurrentDevice(DeviceScratch **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return chd::set_error(CHD_ERR_HIP, std::string("chd_hmult_noalloc: "
                                                   "hipGetDevice: ") +
                                           hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_mu);
  if (dev >= static_cast<int>(g_scratch.size())) g_scratch.resize(dev + 1);
  if (g_scratch[dev] == nullptr) {
    std::unique_ptr<DeviceScratch> d(new DeviceScratch);
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return chd::set_error(CHD_ERR_HIP,
                            std::string("chd_hmult_noalloc: "
                                        "hipGetSymbolAddress: ") +
                                hipGetErrorString(e));
    e = hipEventCreateWithFlags(&d->done, hipEventDisableTiming);
    if (e != hipSuccess)
      return chd::set_error(CHD_ERR_HIP,
                            std::string("chd_hmult_noalloc: "
                                        "hipEventCreateWithFlags: ") +
                                hipGetErrorString(e));
    d->ptr = static_cast<uint32_t *>(p);
    g_scratch[dev] = std::move(d);
  }
  *out = g_scratch[dev].get();
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
  DeviceScratch *ds = nullptr;
  if (int st = ScratchOfCurrentDevice(&ds)) return st;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  std::lock_guard<std::mutex> lock(ds->mu);
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
  const auto key = chd_capi::MakeEvk(ctx, evk_bx, evk_ax, evk_beta);
  // after the previous user of the array, whatever its context or stream
  if (ds->has_last && ds->last != s)
    cheddar::HipCheck(hipStreamWaitEvent(s, ds->done, 0),
                      "hipStreamWaitEvent");
  // this call becomes the array's last user once its kernels are enqueued,
  // also when it throws after some of them
  struct Record {
    DeviceScratch *d;
    hipStream_t s;
    ~Record() {
      if (hipEventRecord(d->done, s) == hipSuccess) {
        d->last = s;
        d->has_last = true;
      } else {
        // no event to order the next call after this one: finish this one
        (void)hipStreamSynchronize(s);
        d->has_last = false;
      }
    }
  };
  {
    Record rec{ds, s};
    cheddar::StreamScope scope(s);
    cheddar::Workspace::Use use(ws);
    cheddar::Workspace::External ext(ws, ds->ptr, kScratchWords);
    ctx->c->HMultV(level, {res_bx, res_ax, nullptr}, {a_bx, a_ax, nullptr},
                   {b_bx, b_ax, nullptr}, key, rescale != 0);
  }
  return chd::check_launch("chd_hmult_noalloc");
  CHD_CATCH("chd_hmult_noalloc")
}
