// Implementation of the C++ host API (see cheddar.h). Every method cites the
// reference function whose semantics it keeps.
#include "cheddar.h"

#include <algorithm>
#include <numeric>
#include <climits>
#include <cmath>
#include <exception>
#include <thread>

#include "cheddar_amd.h"
#include "chd_device.h"
#include "overlap.h"
#include "prime_math.h"

namespace cheddar {

namespace {
thread_local hipStream_t g_stream = nullptr;

void K(int status) {
  if (status != 0) throw Error(chd_last_error());
}

int DivCeil(int a, int b) { return (a + b - 1) / b; }

// ModDown's destination-limb counts (polynomials x limbs) up to which the
// BConv writes the destination and a two-pass NTT runs in place on it; above
// them a single-pass NTT does. The one-source case (Rescale) has its own,
// lower limit: there the single pass forms the BConv itself and saves a
// launch. Measured on MI355X, warm, microseconds (threshold 32 / single pass
// everywhere / two passes everywhere):
//   ModDown, 1 poly, 8..24 limbs: 28.2..33.2 / 32.4..37.8 / 28.2..33.2
//   HMult (merged rescale), 2 x 19 and 2 x 23 limbs: 86.9, 89.0 / 86.8,
//     88.9 / 88.1, 91.2; 2 x 15: 70.4 (two passes) / 70.9 (single)
//   Rescale, 1 poly, 7 / 11 / 15 / 19 / 23 limbs: two passes 25.8 / 27.0 /
//     28.2 / 30.5 / 31.3, single pass 27.6 / 27.5 / 27.7 / 28.1 / 27.8
#ifndef CHD_SMALL_MODDOWN_LIMBS
#define CHD_SMALL_MODDOWN_LIMBS 32
#endif
#ifndef CHD_SMALL_RESCALE_LIMBS
#define CHD_SMALL_RESCALE_LIMBS 12
#endif
// 1: a hoisting handle with a wide giant-step accumulation keeps a tiled
// copy of its plaintexts beside the per-pair ones (twice their memory); 0:
// the accumulation reads the per-pair plaintexts in place
#ifndef CHD_GS_TILED
#define CHD_GS_TILED 1
#endif

chd_limb_map NoSkipMap(const Parameter<uint32_t> &param, const NPInfo &np) {
  chd_limb_map m{};
  m.num_q = np.GetNumQ();
  m.skip_lo = INT_MAX;
  m.skip_len = 0;
  m.tab_off = param.TerLeft(np);
  m.tab_gap = param.MainLeft(np);
  return m;
}
}  // namespace

hipStream_t CurrentStream() { return g_stream; }
StreamScope::StreamScope(hipStream_t s) : prev_(g_stream) { g_stream = s; }
StreamScope::~StreamScope() { g_stream = prev_; }

Workspace::Workspace(size_t words) {
  buf_.Resize(words * sizeof(uint32_t));
  base_ = buf_.as<uint32_t>();
  cap_ = words;
  HipCheck(hipEventCreateWithFlags(&done_, hipEventDisableTiming),
           "hipEventCreateWithFlags");
}

Workspace::~Workspace() {
  if (done_ != nullptr) (void)hipEventDestroy(done_);
}

void Workspace::Enter() {
  mu_.lock();
  if (depth_++ > 0) return;
  cur_ = CurrentStream();
  if (has_last_ && cur_ != last_) {
    const hipError_t e = hipStreamWaitEvent(cur_, done_, 0);
    if (e != hipSuccess) {
      depth_--;
      mu_.unlock();
      HipCheck(e, "hipStreamWaitEvent");
    }
  }
}

void Workspace::Leave() noexcept {
  if (--depth_ == 0) {
    if (hipEventRecord(done_, cur_) == hipSuccess) {
      last_ = cur_;
      has_last_ = true;
    } else {
      // no event to order the next stream after this one: finish the work
      (void)hipStreamSynchronize(cur_);
      has_last_ = false;
    }
  }
  mu_.unlock();
}

Workspace::Use::Use(Workspace *ws) : ws_(ws) {
  if (ws_ != nullptr) ws_->Enter();
}
Workspace::Use::~Use() {
  if (ws_ != nullptr) ws_->Leave();
}

Workspace::External::External(Workspace *ws, uint32_t *base, size_t words)
    : ws_(ws), saved_base_(ws->base_), saved_cap_(ws->cap_) {
  AssertTrue(ws->depth_ > 0 && ws->top_ == 0 && !ws->strict_,
             "Workspace: external memory needs an idle guarded workspace");
  AssertTrue(base != nullptr && (reinterpret_cast<uintptr_t>(base) & 255) == 0,
             "Workspace: external memory must be 256-byte aligned");
  ws->base_ = base;
  ws->cap_ = words & ~static_cast<size_t>(63);
  ws->strict_ = true;
}

Workspace::External::~External() {
  ws_->base_ = saved_base_;
  ws_->cap_ = saved_cap_;
  ws_->top_ = 0;
  ws_->strict_ = false;
}

uint32_t *Workspace::Push(size_t words) {
  const size_t w = (words + 63) & ~static_cast<size_t>(63);  // 256-byte steps
  if (w > cap_ - top_) return nullptr;
  uint32_t *p = base_ + top_;
  top_ += w;
  return p;
}

void Workspace::Pop(uint32_t *p) { top_ = static_cast<size_t>(p - base_); }

Scratch::Scratch(Workspace *ws, size_t words) {
  if (words == 0) return;
  if (ws != nullptr) {
    p_ = ws->Push(words);
    if (p_ != nullptr) {
      ws_ = ws;
      return;
    }
    if (ws->Strict())
      throw Error("ERROR: the temporaries of this call exceed the scratch "
                  "memory it was given");
  }
  s_ = CurrentStream();
  HipCheck(hipMallocAsync(reinterpret_cast<void **>(&p_),
                          words * sizeof(uint32_t), s_),
           "hipMallocAsync");
}

Scratch::~Scratch() {
  if (p_ == nullptr) return;
  if (ws_ != nullptr)
    ws_->Pop(p_);
  else
    (void)hipFreeAsync(p_, s_);
}

NPInfo::NPInfo(int num_main, int num_ter, int num_aux)
    : num_main_(num_main), num_ter_(num_ter), num_aux_(num_aux) {
  AssertTrue(num_main >= 0 && num_ter >= 0 && num_aux >= 0,
             "NPInfo: negative prime count");
}

// ------------------------------------------------------------ Parameter --
// src/core/Parameter.cu:20-194
static int CheckedDnum(size_t main, size_t ter, size_t aux) {
  AssertTrue(aux > 0, "Parameter: at least one auxiliary prime is required");
  return static_cast<int>((main + ter + aux - 1) / aux);
}

Parameter<uint32_t>::Parameter(
    int log_degree, double base_scale, int default_encryption_level,
    std::vector<std::pair<int, int>> level_config,
    const std::vector<word> &main_primes, const std::vector<word> &aux_primes,
    const std::vector<word> &ter_primes,
    const std::pair<int, int> &additional_base)
    : log_degree_(log_degree),
      degree_(1 << log_degree),
      dnum_(CheckedDnum(main_primes.size(), ter_primes.size(),
                        aux_primes.size())),
      L_(static_cast<int>(main_primes.size() + ter_primes.size())),
      alpha_(static_cast<int>(aux_primes.size())),
      base_scale_(base_scale),
      default_encryption_level_(default_encryption_level),
      max_level_(static_cast<int>(level_config.size()) - 1),
      main_primes_(main_primes),
      ter_primes_(ter_primes),
      aux_primes_(aux_primes),
      level_config_(std::move(level_config)) {
  AssertTrue(log_degree == 16, "Parameter: only log_degree 16 is supported");
  AssertTrue(additional_base.first == 0 && additional_base.second == 0,
             "Parameter: additional base (sparse-secret encapsulation) is not "
             "supported by this build");
  AssertTrue(max_level_ >= 0, "Parameter: empty level_config");
  const word ntt_base = 2u * static_cast<word>(degree_);
  auto check = [&](word p) {
    // the reference's own bound check is a no-op (Parameter.cu:45-53);
    // it is enforced here
    AssertTrue(p < (1u << 31), "Max prime is too large for the word size");
    AssertTrue(p % ntt_base == 1, "Prime is not NTT-friendly");
  };
  for (word p : main_primes_) check(p);
  for (word p : aux_primes_) check(p);
  for (word p : ter_primes_) check(p);
  // Parameter.cu:64-91: every level but the last has at most the available
  // primes and more primes than the one below it (or as many, with more
  // main primes); the last holds all of them
  auto below = [](const std::pair<int, int> &a, const std::pair<int, int> &b) {
    const int ta = a.first + a.second, tb = b.first + b.second;
    return ta < tb || (ta == tb && a.first < b.first);
  };
  std::pair<int, int> prev{0, 0};
  for (size_t i = 0; i + 1 < level_config_.size(); i++) {
    const auto &c = level_config_[i];
    AssertTrue(c.first >= 0 && c.first <= GetMaxNumMain(),
               "Invalid number of main primes (" + std::to_string(c.first) +
                   ") at level " + std::to_string(i));
    AssertTrue(c.second >= 0 && c.second <= GetMaxNumTer(),
               "Invalid number of terminal primes (" +
                   std::to_string(c.second) + ") at level " +
                   std::to_string(i));
    AssertTrue(below(prev, c),
               "Invalid level configuration at level " + std::to_string(i));
    prev = c;
  }
  AssertTrue(level_config_.back().first == GetMaxNumMain(),
             "Invalid number of main primes (" +
                 std::to_string(level_config_.back().first) +
                 ") at the last level");
  AssertTrue(level_config_.back().second == GetMaxNumTer(),
             "Invalid number of terminal primes (" +
                 std::to_string(level_config_.back().second) +
                 ") at the last level");
  AssertTrue(default_encryption_level_ >= 0 &&
                 default_encryption_level_ <= max_level_,
             "Invalid default encryption level");
  // galois factors 5^i mod 2N (Parameter.cu:93-101)
  const int slots = degree_ / 2, m = 2 * degree_;
  galois_factors_.resize(slots + 1);
  galois_factors_[0] = 1;
  galois_factors_[slots] = 1;
  for (int i = 1; i < slots; i++)
    galois_factors_[i] = static_cast<int>(
        (static_cast<int64_t>(galois_factors_[i - 1]) * 5) % m);
  chain_.insert(chain_.end(), ter_primes_.rbegin(), ter_primes_.rend());
  chain_.insert(chain_.end(), main_primes_.begin(), main_primes_.end());
  chain_.insert(chain_.end(), aux_primes_.begin(), aux_primes_.end());
  // scales (Parameter.cu:149-193): going down from level i to i - 1 divides
  // by the primes that leave and multiplies by the primes that come back
  rescale_prime_prod_.assign(max_level_ + 1, 0.0);
  scale_.assign(default_encryption_level_ + 1, base_scale_);
  double s = base_scale_;
  for (int i = 1; i <= max_level_; i++) {
    const auto &up = level_config_[i], &lo = level_config_[i - 1];
    double num = 1.0, den = 1.0;
    for (int j = lo.second; j < up.second; j++) num *= ter_primes_[j];
    for (int j = up.second; j < lo.second; j++) den *= ter_primes_[j];
    for (int j = lo.first; j < up.first; j++) num *= main_primes_[j];
    for (int j = up.first; j < lo.first; j++) den *= main_primes_[j];
    const double prod = num / den;
    rescale_prime_prod_[i] = prod;
    if (i <= default_encryption_level_) {
      s = std::sqrt(s * prod);
      scale_[i] = s;
    }
  }
}

NPInfo Parameter<uint32_t>::LevelToNP(int level, int num_aux) const {
  AssertTrue(num_aux >= 0 && num_aux <= alpha_, "Invalid number of aux primes");
  AssertTrue(level >= 0 && level <= max_level_, "Invalid level");
  const auto &c = level_config_.at(level);
  return NPInfo(c.first, c.second, num_aux);
}

// Parameter.cu:297-313 (the levels are ordered, so the first match is the
// one its binary search finds)
int Parameter<uint32_t>::NPToLevel(const NPInfo &np) const {
  for (size_t i = 0; i < level_config_.size(); i++)
    if (level_config_[i].first == np.num_main_ &&
        level_config_[i].second == np.num_ter_)
      return static_cast<int>(i);
  Fail("NPInfo not found");
}

std::vector<uint32_t> Parameter<uint32_t>::GetPrimeVector(
    const NPInfo &np) const {
  std::vector<word> r(chain_.begin() + TerLeft(np),
                      chain_.begin() + GetMaxNumTer() + np.num_main_);
  r.insert(r.end(), aux_primes_.begin(), aux_primes_.begin() + np.num_aux_);
  return r;
}

int Parameter<uint32_t>::GetGaloisFactor(int i) const {
  AssertTrue(i >= 0 && i <= degree_ / 2,
             "GetGaloisFactor: Invalid Galois factor index");
  return galois_factors_.at(i);
}

double Parameter<uint32_t>::GetScale(int level) const {
  AssertTrue(level >= 0 && level <= default_encryption_level_,
             "GetScale: Invalid level");
  return scale_.at(level);
}

double Parameter<uint32_t>::GetRescalePrimeProd(int level) const {
  AssertTrue(level > 0 && level <= max_level_,
             "GetRescalePrimeProd: Invalid level");
  return rescale_prime_prod_.at(level);
}

// ----------------------------------------------------------- containers --
Ciphertext<uint32_t>::Ciphertext(const NPInfo &np, bool has_rx) : np_(np) {
  size_t n = static_cast<size_t>(np.GetNumTotal()) * degree_;
  bx_.resize(n);
  ax_.resize(n);
  if (has_rx) rx_.resize(n);
}

void Ciphertext<uint32_t>::PrepareRx() {
  rx_.resize(static_cast<size_t>(np_.GetNumTotal()) * degree_);
}

void Ciphertext<uint32_t>::RemoveRx() { rx_.resize(0); }

void Ciphertext<uint32_t>::ModifyNP(const NPInfo &np) {
  np_ = np;
  size_t n = static_cast<size_t>(np.GetNumTotal()) * degree_;
  bx_.resize(n);
  ax_.resize(n);
  if (rx_.size() != 0) rx_.resize(n);
}

EvaluationKey<uint32_t>::EvaluationKey(const NPInfo &np, int beta, int degree)
    : np_(np) {
  AssertTrue(beta >= 0, "Negative beta given for evaluation key");
  size_t n = static_cast<size_t>(np.GetNumTotal()) * degree;
  bx_.resize(beta);
  ax_.resize(beta);
  for (int i = 0; i < beta; i++) {
    bx_[i].resize(n);
    ax_[i].resize(n);
  }
}

Plaintext<uint32_t>::Plaintext(const NPInfo &np, int degree) : np_(np) {
  mx_.resize(static_cast<size_t>(np.GetNumTotal()) * degree);
}

Constant<uint32_t>::Constant(const NPInfo &np) : np_(np) {
  cx_.resize(static_cast<size_t>(np.GetNumTotal()));
}

// EvkMap.cpp: GetRotationKey asserts the key exists
const EvaluationKey<uint32_t> &EvkMap<uint32_t>::GetRotationKey(
    int rot_idx) const {
  auto it = find(rot_idx);
  AssertTrue(it != end(),
             "EvkMap: rotation key " + std::to_string(rot_idx) + " not found");
  return it->second;
}

// ------------------------------------------------------------ NTTHandler --
NTTHandler<uint32_t>::NTTHandler(const Parameter<word> &param)
    : param_(param), chain_(param.log_degree_, param.ChainPrimes()) {}

chd_limb_map NTTHandler<uint32_t>::Map(const NPInfo &np) const {
  return NoSkipMap(param_, np);
}

namespace {
// Limb gap between src's q and aux parts, checked against src's size: the
// kernels read num_q limbs from src and num_aux limbs from src + QSize().
int SrcGap(const DvConstView<uint32_t> &src, const NPInfo &np, int n,
           const char *who) {
  AssertTrue(src.QSize() >= np.GetNumQ() * n && src.QSize() % n == 0 &&
                 src.TotalSize() >= src.QSize() + np.num_aux_ * n,
             std::string(who) + ": src too small for its limbs");
  return (src.QSize() - np.GetNumQ() * n) / n;
}
}  // namespace

// src/core/NTT.cu:606-671
void NTTHandler<uint32_t>::NTT(DvView<word> &dst, const NPInfo &np,
                               const DvConstView<word> &src,
                               bool montgomery_conversion) const {
  const int n = param_.degree_;
  AssertTrue(dst.TotalSize() == np.GetNumTotal() * n, "NTT: Invalid dst size");
  chd_limb_map m = Map(np);
  m.src_gap = SrcGap(src, np, n, "NTT");
  m.cst_gap = param_.MainLeft(np);
  const word *pre = montgomery_conversion
                        ? chain_.mont_converter() + param_.TerLeft(np)
                        : nullptr;
  K(chd_k_ntt_fwd(&chain_.tables(), &m, dst.data(), 0, src.data(), 0,
                  np.GetNumTotal(), 1, pre, CurrentStream()));
}

// src/core/NTT.cu:673-741
void NTTHandler<uint32_t>::INTT(DvView<word> &dst, const NPInfo &np,
                                const DvConstView<word> &src,
                                bool montgomery_conversion) const {
  const int n = param_.degree_;
  AssertTrue(dst.TotalSize() == np.GetNumTotal() * n,
             "INTT: Invalid dst size");
  chd_limb_map m = Map(np);
  m.src_gap = SrcGap(src, np, n, "INTT");
  m.cst_gap = param_.MainLeft(np);
  const word *cst =
      (montgomery_conversion ? chain_.inv_degree() : chain_.inv_degree_mont()) +
      param_.TerLeft(np);
  K(chd_k_ntt_inv(&chain_.tables(), &m, dst.data(), 0, src.data(), 0,
                  np.GetNumTotal(), 1, cst, 0, CurrentStream()));
}

// src/core/NTT.cu:743-813
void NTTHandler<uint32_t>::INTTAndMultConst(DvView<word> &dst,
                                            const NPInfo &np,
                                            const DvConstView<word> &src,
                                            const DvConstView<word> &src_const,
                                            bool normalize) const {
  const int n = param_.degree_;
  AssertTrue(dst.TotalSize() == np.GetNumTotal() * n,
             "INTTAndMultConst: Invalid dst size");
  AssertTrue(src_const.QSize() >= np.GetNumQ() &&
                 src_const.TotalSize() >= src_const.QSize() + np.num_aux_,
             "INTTAndMultConst: src_const too small for its limbs");
  chd_limb_map m = Map(np);
  m.src_gap = SrcGap(src, np, n, "INTTAndMultConst");
  m.cst_gap = src_const.QSize() - np.GetNumQ();
  K(chd_k_ntt_inv(&chain_.tables(), &m, dst.data(), 0, src.data(), 0,
                  np.GetNumTotal(), 1, src_const.data(), normalize ? 1 : 0,
                  CurrentStream()));
}

// src/core/NTT.cu:815-887
void NTTHandler<uint32_t>::NTTForModUp(DvView<word> &dst, const NPInfo &np,
                                       int skip_start, int skip_end,
                                       const DvConstView<word> &src) const {
  const int n = param_.degree_;
  const int num_q = np.GetNumQ();
  AssertTrue(dst.TotalSize() == np.GetNumTotal() * n,
             "NTTForModUp: Invalid dst size");
  AssertTrue(skip_start >= 0 && skip_start < num_q && skip_end >= skip_start &&
                 skip_end <= num_q,
             "NTTForModUp: Invalid skip primes");
  chd_limb_map m = Map(np);
  m.skip_lo = skip_start;
  m.skip_len = skip_end - skip_start;
  m.src_gap = SrcGap(src, np, n, "NTTForModUp");
  K(chd_k_ntt_fwd(&chain_.tables(), &m, dst.data(), 0, src.data(), 0,
                  np.GetNumTotal() - m.skip_len, 1, nullptr, CurrentStream()));
}

// src/core/NTT.cu:889-971 (kFuseModDownEpilogue, kFuseMontgomery)
void NTTHandler<uint32_t>::NTTForModDown(
    DvView<word> &dst, const NPInfo &np_src1, const NPInfo &np_src2,
    const DvConstView<word> &src1, const DvConstView<word> &src2,
    const DvConstView<word> &inv_p_prod,
    const DvConstView<word> &src2_padding) const {
  const int n = param_.degree_;
  const int total = np_src1.GetNumTotal();
  AssertTrue(dst.TotalSize() == total * n, "NTTForModDown: Invalid dst size");
  AssertTrue(np_src1.num_aux_ == 0, "NTTForModDown: num_aux should be 0");
  AssertTrue(np_src2.GetNumQ() <= total, "NTTForModDown: Invalid src2 size");
  AssertTrue(dst.data() != src2.data(),
             "NTTForModDown: dst and src2 should be different");
  AssertTrue(src1.data() == dst.data(),
             "NTTForModDown: src1 must be dst (in-place NTT)");
  const int s2_lo = np_src1.num_ter_ - np_src2.num_ter_;
  const int s2_hi = s2_lo + np_src2.GetNumQ();
  AssertTrue(s2_hi <= total, "NTTForModDown: Invalid src2 size");
  chd_limb_map m = Map(np_src1);
  K(chd_k_ntt_fwd_moddown(&chain_.tables(), &m, dst.data(), total,
                          src2.data(), s2_lo, s2_hi, inv_p_prod.data(),
                          src2_padding.data(), CurrentStream()));
}

// src/core/NTT.cu:973-1071 (case 1: INTT on the upper part only)
void NTTHandler<uint32_t>::INTTForModDown(
    DvView<word> &dst, const NPInfo &np_src, const NPInfo &np_non_intt,
    const DvConstView<word> &src, const DvConstView<word> &src_const) const {
  const int n = param_.degree_;
  const int limbs = np_src.GetNumTotal() - np_non_intt.GetNumTotal();
  AssertTrue(dst.TotalSize() == limbs * n, "INTTForModDown: Invalid dst size");
  AssertTrue(np_src.GetNumQ() * n == src.QSize() &&
                 np_src.GetNumTotal() * n == src.TotalSize(),
             "INTTForModDown: Invalid src size");
  AssertTrue(np_non_intt.num_aux_ == 0 && np_non_intt.IsSubsetOf(np_src),
             "INTTForModDown: Invalid np combination");
  AssertTrue(src.data() != dst.data(),
             "INTTForModDown: src and dst should be different");
  AssertTrue(src_const.TotalSize() == limbs,
             "INTTForModDown: Invalid src_const size");
  AssertTrue(np_src.num_ter_ == np_non_intt.num_ter_,
             "INTTForModDown: terminal-prime INTT is not supported");
  chd_limb_map m{};
  m.num_q = np_src.num_main_ - np_non_intt.num_main_;
  m.skip_lo = INT_MAX;
  m.tab_off = param_.GetMaxNumTer() + np_non_intt.num_main_;
  m.tab_gap = param_.MainLeft(np_src);
  const size_t off =
      static_cast<size_t>(np_src.num_ter_ + np_non_intt.num_main_) * n;
  K(chd_k_ntt_inv(&chain_.tables(), &m, dst.data(), 0, src.data() + off, 0,
                  limbs, 1, src_const.data(), 1, CurrentStream()));
}

// --------------------------------------------------- ElementWiseHandler --
ElementWiseHandler<uint32_t>::ElementWiseHandler(const Parameter<word> &param,
                                                 const NTTHandler<word> &ntt)
    : param_(param), ntt_(ntt) {}

// src/core/ElementWise.cu:921-953
void ElementWiseHandler<uint32_t>::Tensor(
    std::vector<DvView<word>> &dst, const NPInfo &np,
    const std::vector<DvConstView<word>> &src1,
    const std::vector<DvConstView<word>> &src2) const {
  AssertTrue(dst.size() == 3 && src1.size() == 2 && src2.size() == 2,
             "Tensor: Invalid number of polynomials");
  const int n = param_.degree_;
  const int q_size = np.GetNumQ() * n;
  for (auto &d : dst)
    AssertTrue(d.TotalSize() == np.GetNumTotal() * n, "Tensor: NP mismatch");
  chd_limb_map m = NoSkipMap(param_, np);
  m.src_gap = (src1[0].QSize() - q_size) / n;
  AssertTrue(np.num_aux_ == 0 ||
                 src2[0].QSize() - q_size == src1[0].QSize() - q_size,
             "Tensor: source gap mismatch");
  K(chd_k_tensor(&ntt_.Tables(), &m, dst[0].data(), dst[1].data(),
                 dst[2].data(), src1[0].data(), src1[1].data(), src2[0].data(),
                 src2[1].data(), np.GetNumTotal(), CurrentStream()));
}

// src/core/ElementWise.cu:1437-1643
void ElementWiseHandler<uint32_t>::CPAccumWorker(
    bool const_accum, std::vector<DvView<word>> &dst, const NPInfo &np,
    const std::vector<std::vector<DvConstView<word>>> &ct_srcs,
    const std::vector<DvConstView<word>> &common_srcs) const {
  const int num_poly = static_cast<int>(dst.size());
  const int num_accum = static_cast<int>(common_srcs.size());
  const bool has_extra_ct = ct_srcs.size() == common_srcs.size() + 1;
  AssertTrue(num_poly > 0 && num_poly <= CHD_MAX_POLY,
             "CPAccum: Invalid number of polynomials");
  AssertTrue(num_accum == static_cast<int>(ct_srcs.size()) || has_extra_ct,
             "CPAccum: Incompatible ct_srcs/common_srcs size");
  AssertTrue(num_accum > 0, "CPAccum: Invalid number of accumulations");
  const int n = param_.degree_;
  const int q_size = np.GetNumQ() * n;
  for (auto &d : dst)
    AssertTrue(d.TotalSize() == np.GetNumTotal() * n, "CPAccum: NP mismatch");
  for (auto &c : ct_srcs)
    AssertTrue(static_cast<int>(c.size()) == num_poly,
               "CPAccum: Incompatible dst/ct_src size");
  chd_limb_map m = NoSkipMap(param_, np);
  std::vector<uint32_t *> dptr(num_poly);
  for (int p = 0; p < num_poly; p++) dptr[p] = dst[p].data();
  std::vector<const uint32_t *> s0(num_poly);
  long long s0_gap = 0;
  bool use_s0 = has_extra_ct;
  if (has_extra_ct) {
    for (int p = 0; p < num_poly; p++) s0[p] = ct_srcs.back()[p].data();
    s0_gap = ct_srcs.back()[0].QSize() - q_size;
  }
  // accumulate in chunks of CHD_MAX_ACCUM; later chunks add onto dst
  for (int base = 0; base < num_accum; base += CHD_MAX_ACCUM) {
    const int cnt = std::min(CHD_MAX_ACCUM, num_accum - base);
    chd_accum_src s[CHD_MAX_ACCUM] = {};
    for (int j = 0; j < cnt; j++) {
      const auto &ct = ct_srcs[base + j];
      const auto &cm = common_srcs[base + j];
      for (int p = 0; p < num_poly; p++) s[j].src[p] = ct[p].data();
      s[j].src_gap = ct[0].QSize() - q_size;
      s[j].common = cm.data();
      s[j].common_gap =
          const_accum ? cm.QSize() - np.GetNumQ() : cm.QSize() - q_size;
    }
    K(chd_k_cpaccum(&ntt_.Tables(), &m, dptr.data(), num_poly,
                    use_s0 ? s0.data() : nullptr, s0_gap, s, cnt,
                    const_accum ? 1 : 0, np.GetNumTotal(), CurrentStream()));
    for (int p = 0; p < num_poly; p++) s0[p] = dptr[p];
    s0_gap = 0;
    use_s0 = true;
  }
}

void ElementWiseHandler<uint32_t>::PAccum(
    std::vector<DvView<word>> &dst, const NPInfo &np,
    const std::vector<std::vector<DvConstView<word>>> &ct_srcs,
    const std::vector<DvConstView<word>> &common_srcs) const {
  CPAccumWorker(false, dst, np, ct_srcs, common_srcs);
}

void ElementWiseHandler<uint32_t>::CAccum(
    std::vector<DvView<word>> &dst, const NPInfo &np,
    const std::vector<std::vector<DvConstView<word>>> &ct_srcs,
    const std::vector<DvConstView<word>> &common_srcs) const {
  CPAccumWorker(true, dst, np, ct_srcs, common_srcs);
}

// src/core/ElementWise.cu:955-964
uint32_t ElementWiseHandler<uint32_t>::PermuteAmountToGaloisFactor(
    int permute_amount) const {
  if (permute_amount == -1) return 2u * param_.degree_ - 1;
  AssertTrue(permute_amount >= 0 && permute_amount <= param_.degree_ / 2,
             "Permute: Invalid permute amount");
  return static_cast<uint32_t>(param_.GetGaloisFactor(permute_amount));
}

// src/core/ElementWise.cu:966-999
void ElementWiseHandler<uint32_t>::Permute(
    std::vector<DvView<word>> &dst, const NPInfo &np, int permute_amount,
    const std::vector<DvConstView<word>> &src1) const {
  const int num_poly = static_cast<int>(dst.size());
  AssertTrue(num_poly == static_cast<int>(src1.size()),
             "Permute: Incompatible dst/src size");
  AssertTrue(num_poly > 0 && num_poly <= CHD_MAX_POLY,
             "Permute: Invalid number of polynomials");
  const int n = param_.degree_;
  std::vector<uint32_t *> d(num_poly);
  std::vector<const uint32_t *> s(num_poly);
  for (int p = 0; p < num_poly; p++) {
    AssertTrue(dst[p].data() != src1[p].data(),
               "Permute does not support inplace operation");
    d[p] = dst[p].data();
    s[p] = src1[p].data();
  }
  chd_limb_map m = NoSkipMap(param_, np);
  m.src_gap = (src1[0].QSize() - np.GetNumQ() * n) / n;
  K(chd_k_permute(&m, d.data(), s.data(), num_poly, np.GetNumTotal(),
                  PermuteAmountToGaloisFactor(permute_amount),
                  CurrentStream()));
}

// ElementWise.cu:1002-1110 (PermuteAccumWorker): one launch per
// CHD_MAX_ACCUM sources; later launches add onto dst
void ElementWiseHandler<uint32_t>::PermuteAccum(
    std::vector<DvView<word>> &dst, const NPInfo &np,
    const std::vector<int> &permute_amounts,
    const std::vector<std::vector<DvConstView<word>>> &srcs) const {
  const int num_poly = static_cast<int>(dst.size());
  const int num_accum = static_cast<int>(permute_amounts.size());
  const bool has_extra_ct = static_cast<int>(srcs.size()) == num_accum + 1;
  AssertTrue(num_poly > 0 && num_poly <= CHD_MAX_POLY,
             "PermuteAccum: Invalid number of polynomials");
  AssertTrue(num_accum == static_cast<int>(srcs.size()) || has_extra_ct,
             "PermuteAccum: Incompatible srcs/permute_amounts size");
  AssertTrue(num_accum > 0 || has_extra_ct,
             "PermuteAccum: nothing to accumulate");
  const int n = param_.degree_;
  const int q_size = np.GetNumQ() * n;
  for (auto &d : dst)
    AssertTrue(d.TotalSize() == np.GetNumTotal() * n,
               "PermuteAccum: NP mismatch");
  for (auto &s : srcs)
    AssertTrue(static_cast<int>(s.size()) == num_poly,
               "PermuteAccum: Incompatible dst/src size");
  chd_limb_map m = NoSkipMap(param_, np);
  std::vector<uint32_t *> dptr(num_poly);
  std::vector<const uint32_t *> s0(num_poly);
  for (int p = 0; p < num_poly; p++) dptr[p] = dst[p].data();
  bool use_s0 = has_extra_ct;
  long long s0_gap = 0;
  if (has_extra_ct) {
    for (int p = 0; p < num_poly; p++) s0[p] = srcs.back()[p].data();
    s0_gap = srcs.back()[0].QSize() - q_size;
  }
  // a source that aliases dst would be read after other blocks wrote it
  for (int j = 0; j < num_accum; j++)
    for (int p = 0; p < num_poly; p++)
      AssertTrue(srcs[j][p].data() != dptr[p] || permute_amounts[j] == 0,
                 "PermuteAccum: a permuted source cannot alias dst");
  int base = 0;
  do {
    const int cnt = std::min(CHD_MAX_ACCUM, num_accum - base);
    chd_perm_src s[CHD_MAX_ACCUM] = {};
    for (int j = 0; j < cnt; j++) {
      for (int p = 0; p < num_poly; p++) s[j].src[p] = srcs[base + j][p].data();
      s[j].src_gap = srcs[base + j][0].QSize() - q_size;
      s[j].galois = PermuteAmountToGaloisFactor(permute_amounts[base + j]);
    }
    K(chd_k_permute_accum(&ntt_.Tables(), &m, dptr.data(), num_poly,
                          use_s0 ? s0.data() : nullptr, s0_gap, s, cnt,
                          np.GetNumTotal(), CurrentStream()));
    for (int p = 0; p < num_poly; p++) s0[p] = dptr[p];
    s0_gap = 0;
    use_s0 = true;
    base += cnt;
  } while (base < num_accum);
}

// ----------------------------------------------------- ModSwitchHandler --
// src/core/ModSwitch.cu:175-318
ModSwitchHandler<uint32_t>::ModSwitchHandler(
    const Parameter<word> &param, int level,
    const ElementWiseHandler<word> &elem, const NTTHandler<word> &ntt,
    Workspace *ws)
    : level_(level),
      num_aux_(param.alpha_),
      beta_(DivCeil(param.LevelToNP(level).num_main_ + param.GetMaxNumTer(),
                    param.alpha_)),
      prime_offset_(param.GetMaxNumTer() - param.LevelToNP(level).num_ter_),
      first_group_(prime_offset_ / param.alpha_),
      group_shift_(prime_offset_ % param.alpha_),
      param_(param),
      ntt_(ntt),
      ws_(ws) {
  // the reference's constructor also takes the element-wise handler; this
  // one keeps none of its state
  (void)elem;
  const NPInfo np = param_.LevelToNP(level_, num_aux_);
  const int num_q = np.GetNumQ();
  const std::vector<word> lp = param_.GetPrimeVector(np);
  // ModUp constants per non-empty group (ModSwitch.cu:200-235)
  std::vector<word> up1(num_q);
  mod_up_.resize(NumGroups());
  for (int z = 0; z < NumGroups(); z++) {
    const int s0 = GroupLo(z), s1 = GroupHi(z);
    std::vector<word> src(lp.begin() + s0, lp.begin() + s1);
    std::vector<word> dst(lp.begin(), lp.begin() + s0);
    dst.insert(dst.end(), lp.begin() + s1, lp.end());
    BuildSwitch(mod_up_[z], src, dst);
    std::vector<word> c1(s1 - s0);
    HipCheck(hipMemcpy(c1.data(), mod_up_[z].const1.data(),
                       c1.size() * sizeof(word), hipMemcpyDeviceToHost),
             "hipMemcpy");
    std::copy(c1.begin(), c1.end(), up1.begin() + s0);
  }
  mod_up1_.resize(num_q);
  HipCheck(hipMemcpy(mod_up1_.data(), up1.data(), num_q * sizeof(word),
                     hipMemcpyHostToDevice),
           "hipMemcpy");

  const std::vector<word> qp(lp.begin(), lp.begin() + num_q);
  const std::vector<word> pp(lp.begin() + num_q, lp.end());
  BuildSwitch(mod_down_, pp, qp);
  auto inv_prod = [](const std::vector<word> &src,
                     const std::vector<word> &dst) {
    std::vector<word> r(dst.size());
    for (size_t k = 0; k < dst.size(); k++) {
      word v = 1;
      for (word s : src) v = pm::mulmod(v, s % dst[k], dst[k]);
      r[k] = pm::to_mont(pm::invmod(v, dst[k]), dst[k]);
    }
    return r;
  };
  auto upload = [](DeviceVector<word> &dv, const std::vector<word> &h) {
    dv.resize(h.size());
    HipCheck(hipMemcpy(dv.data(), h.data(), h.size() * sizeof(word),
                       hipMemcpyHostToDevice),
             "hipMemcpy");
  };
  upload(inv_prime_prod_, inv_prod(pp, qp));
  if (level_ == 0) return;

  // Rescale constants (ModSwitch.cu:252-318): the primes that leave, and
  // the BitPacker restore range of the primes that come back
  const NPInfo next = param_.LevelToNP(level_ - 1);
  const std::vector<word> rdst = param_.GetPrimeVector(next);
  const int next_q = next.GetNumQ();
  const int main_diff = np.num_main_ - next.num_main_;
  const int ter_diff = np.num_ter_ - next.num_ter_;
  std::vector<word> rsrc;
  int rlo = 0, rhi = 0;
  if (ter_diff > 0) {  // terminal primes leave, main primes may come back
    AssertTrue(main_diff <= 0, "Invalid rescale amount");
    rsrc.assign(lp.begin(), lp.begin() + ter_diff);
    rlo = next_q + main_diff;
    rhi = next_q;
  } else if (main_diff > 0) {  // main primes leave, terminal may come back
    AssertTrue(ter_diff <= 0, "Invalid rescale amount");
    rsrc.assign(lp.begin() + num_q - main_diff, lp.begin() + num_q);
    rlo = 0;
    rhi = -ter_diff;
  } else {
    Fail("Invalid rescale amount");
  }
  std::vector<word> mdr_src = rsrc;
  mdr_src.insert(mdr_src.end(), pp.begin(), pp.end());
  BuildSwitch(rescale_, rsrc, rdst, rlo, rhi);
  BuildSwitch(mod_down_rescale_, mdr_src, rdst, rlo, rhi);
  upload(rescale_inv_prime_prod_, inv_prod(rsrc, rdst));
  upload(mod_down_rescale_inv_prime_prod_, inv_prod(mdr_src, rdst));
  if (rhi > rlo) {
    // padding of the kept limbs, indexed as src2 (ModSwitch.cu:388-411):
    // ToMont(prod of the restored primes)
    const int rlen = rhi - rlo;
    std::vector<word> pad(next_q - rlen);
    for (int i = 0; i < next_q - rlen; i++) {
      const word m = rdst[i >= rlo ? i + rlen : i];
      word v = 1;
      for (int j = rlo; j < rhi; j++) v = pm::mulmod(v, rdst[j] % m, m);
      pad[i] = pm::to_mont(v, m);
    }
    upload(rescale_padding_, pad);
    upload(mod_down_rescale_padding_, pad);
  }
}

int ModSwitchHandler<uint32_t>::GroupLo(int z) const {
  return chd::group_lo(z, num_aux_, group_shift_);
}

int ModSwitchHandler<uint32_t>::GroupHi(int z) const {
  return chd::group_hi(z, num_aux_, group_shift_,
                       param_.LevelToNP(level_).GetNumQ());
}

// PopulateModSwitchConstants (ModSwitch.cu:320-370)
void ModSwitchHandler<uint32_t>::BuildSwitch(
    SwitchTable &st, const std::vector<word> &src,
    const std::vector<word> &dst, int restore_lo, int restore_hi) const {
  const int sl = static_cast<int>(src.size());
  const int dl = static_cast<int>(dst.size());
  std::vector<word> c1;
  std::vector<int32_t> c2;
  pm::modswitch_constants(src, dst, static_cast<word>(param_.degree_),
                          restore_lo, restore_hi, &c1, &c2);
  st.src_len = sl;
  st.dst_len = dl;
  st.const1.resize(sl);
  HipCheck(hipMemcpy(st.const1.data(), c1.data(), sl * sizeof(word),
                     hipMemcpyHostToDevice),
           "hipMemcpy");
  std::vector<unsigned char> packed(
      static_cast<size_t>(chd_bconv_table_size(sl, dl)));
  K(chd_bconv_table_pack(packed.data(), c2.data(), dst.data(), sl, dl));
  st.table.Resize(packed.size());
  st.table.Upload(packed.data(), packed.size());
  if (sl == 1) {
    std::vector<word> col(dl);
    for (int k = 0; k < dl; k++)
      col[k] = c2[k] < 0 ? static_cast<word>(c2[k] + static_cast<int64_t>(dst[k]))
                         : static_cast<word>(c2[k]);
    st.bconv1.resize(dl);
    HipCheck(hipMemcpy(st.bconv1.data(), col.data(), dl * sizeof(word),
                       hipMemcpyHostToDevice),
             "hipMemcpy");
  }
}

// src/core/ModSwitch.cu:429-485: INTTAndMultConst(centre) of src into intt,
// then the BConv of every dnum group in one launch, group i into dst[i].
void ModSwitchHandler<uint32_t>::ModUpBconv(word *const *dst,
                                            const DvConstView<word> &src,
                                            word *intt,
                                            const word *src_mul) const {
  const NPInfo np = param_.LevelToNP(level_, 0);
  const int num_q = np.GetNumQ();
  const int n = param_.degree_;
  AssertTrue(src.QSize() == num_q * n, "ModUp src q size mismatch");
  AssertTrue(src.AuxSize() == 0, "ModUp src aux size mismatch");
  AssertTrue(NumGroups() <= CHD_MAX_JOBS, "ModUp: dnum larger than supported");
  if (src_mul != nullptr) {
    const chd_limb_map mi = NoSkipMap(param_, np);
    K(chd_k_ntt_inv_mul(&ntt_.Tables(), &mi, intt, 0, src.data(), src_mul, 0,
                        num_q, 1, mod_up1_.data(), 1, CurrentStream()));
  } else {
    DvView<word> intt_view(intt, num_q * n, 0);
    ntt_.INTTAndMultConst(intt_view, np, src,
                          DvConstView<word>(mod_up1_.data(), num_q, 0), true);
  }
  NPInfo np_aux = np;
  np_aux.num_aux_ = num_aux_;
  chd_limb_map m = NoSkipMap(param_, np_aux);
  chd_bconv_job jobs[CHD_MAX_JOBS] = {};
  for (int z = 0; z < NumGroups(); z++) {
    const int s0 = GroupLo(z), s1 = GroupHi(z);
    const SwitchTable &st = mod_up_[z];
    jobs[z].dst = dst[z];
    jobs[z].src = reinterpret_cast<const int32_t *>(intt) +
                  static_cast<size_t>(s0) * n;
    jobs[z].table = st.table.as<void>();
    jobs[z].src_len = st.src_len;
    jobs[z].dst_len = st.dst_len;
    jobs[z].skip_lo = s0;
    jobs[z].skip_len = s1 - s0;
  }
  K(chd_k_bconv_batch(&ntt_.Tables(), &m, jobs, NumGroups(), CurrentStream()));
}

// ModUp with every group's column pass (and, with_rows, row pass) batched;
// group i lives at modup + i * group_stride. Own limbs are not written.
void ModSwitchHandler<uint32_t>::ModUpGroups(word *modup,
                                             long long group_stride,
                                             const DvConstView<word> &src,
                                             word *intt, bool with_rows,
                                             const word *src_mul) const {
  const NPInfo np = param_.LevelToNP(level_, 0);
  const int num_q = np.GetNumQ();
  word *dst[CHD_MAX_JOBS];
  AssertTrue(NumGroups() <= CHD_MAX_JOBS, "ModUp: dnum larger than supported");
  for (int z = 0; z < NumGroups(); z++) dst[z] = modup + z * group_stride;
  ModUpBconv(dst, src, intt, src_mul);
  NPInfo np_aux = np;
  np_aux.num_aux_ = num_aux_;
  chd_limb_map m = NoSkipMap(param_, np_aux);
  K(chd_k_ntt_fwd_groups(&ntt_.Tables(), &m, modup, group_stride, NumGroups(),
                         num_aux_, group_shift_, num_q + num_aux_,
                         with_rows ? 1 : 0, CurrentStream()));
}

void ModSwitchHandler<uint32_t>::ModUpGroupsBatch(word *modup,
                                                  long long group_stride,
                                                  const word *src,
                                                  long long src_stride,
                                                  int num_inputs,
                                                  word *intt) const {
  const NPInfo np = param_.LevelToNP(level_, 0);
  const int num_q = np.GetNumQ();
  const int n = param_.degree_;
  const int groups = NumGroups();
  AssertTrue(num_inputs >= 1 && num_inputs <= CHD_MAX_JOBS,
             "ModUp: 1 to CHD_MAX_JOBS inputs per batch");
  AssertTrue(groups * num_inputs <= CHD_MAX_BCONV_JOBS,
             "ModUp: too many groups in one batch");
  // INTTAndMultConst(centre) of every input (ModSwitch.cu:442-447)
  const chd_limb_map mi = NoSkipMap(param_, np);
  const long long ilen = static_cast<long long>(num_q) * n;
  K(chd_k_ntt_inv(&ntt_.Tables(), &mi, intt, ilen, src, src_stride, num_q,
                  num_inputs, mod_up1_.data(), 1, CurrentStream()));
  NPInfo np_aux = np;
  np_aux.num_aux_ = num_aux_;
  chd_limb_map m = NoSkipMap(param_, np_aux);
  chd_bconv_job jobs[CHD_MAX_BCONV_JOBS] = {};
  for (int i = 0; i < num_inputs; i++)
    for (int z = 0; z < groups; z++) {
      const int s0 = GroupLo(z), s1 = GroupHi(z);
      const SwitchTable &st = mod_up_[z];
      chd_bconv_job &jb = jobs[i * groups + z];
      jb.dst = modup + (static_cast<long long>(i) * groups + z) * group_stride;
      jb.src = reinterpret_cast<const int32_t *>(intt) + i * ilen +
               static_cast<size_t>(s0) * n;
      jb.table = st.table.as<void>();
      jb.src_len = st.src_len;
      jb.dst_len = st.dst_len;
      jb.skip_lo = s0;
      jb.skip_len = s1 - s0;
    }
  K(chd_k_bconv_batch(&ntt_.Tables(), &m, jobs, groups * num_inputs,
                      CurrentStream()));
  K(chd_k_ntt_fwd_groups_batch(&ntt_.Tables(), &m, modup, group_stride,
                               groups, num_inputs, num_aux_, group_shift_,
                               num_q + num_aux_, 0, CurrentStream()));
}

// src/core/ModSwitch.cu:429-509
void ModSwitchHandler<uint32_t>::ModUp(std::vector<DvView<word>> &dst,
                                       const DvConstView<word> &src) const {
  const NPInfo np = param_.LevelToNP(level_, 0);
  const int num_q = np.GetNumQ();
  const int n = param_.degree_;
  AssertTrue(static_cast<int>(dst.size()) == beta_, "ModUp dst size mismatch");
  AssertTrue(NumGroups() <= CHD_MAX_JOBS, "ModUp: dnum larger than supported");
  const long long gs = static_cast<long long>(num_q + num_aux_) * n;
  const int first = first_group_;
  bool strided = true;
  for (int z = 0; z < NumGroups(); z++) {
    const DvView<word> &d = dst[first + z];
    AssertTrue(d.AuxSize() == num_aux_ * n && d.QSize() == num_q * n,
               "ModUp dst size mismatch");
    strided = strided && d.data() == dst[first].data() + z * gs;
  }
  // own limbs are the input's (ModSwitch.cu:449-470); groups before
  // FirstGroup() hold no limb of this level and are not written
  for (int z = 0; z < NumGroups(); z++) {
    const int s0 = GroupLo(z), s1 = GroupHi(z);
    HipCheck(hipMemcpyAsync(dst[first + z].data() + static_cast<size_t>(s0) * n,
                            src.data() + static_cast<size_t>(s0) * n,
                            static_cast<size_t>(s1 - s0) * n * sizeof(word),
                            hipMemcpyDeviceToDevice, CurrentStream()),
             "hipMemcpyAsync");
  }
  Workspace::Use use_ws(ws_);
  Scratch intt(ws_, static_cast<size_t>(num_q) * n);
  if (strided) {  // groups equally spaced: one launch per pass for all
    ModUpGroups(dst[first].data(), gs, src, intt.data(), true);
    return;
  }
  word *d[CHD_MAX_JOBS];
  for (int z = 0; z < NumGroups(); z++) d[z] = dst[first + z].data();
  ModUpBconv(d, src, intt.data());
  NPInfo np_aux = np;
  np_aux.num_aux_ = num_aux_;
  for (int z = 0; z < NumGroups(); z++)
    ntt_.NTTForModUp(dst[first + z], np_aux, GroupLo(z), GroupHi(z),
                     DvConstView<word>(dst[first + z]));
}

// src/core/ModSwitch.cu:414-428 (MultConst by p_prod)
void ModSwitchHandler<uint32_t>::PseudoModUp(
    DvView<word> &dst, const DvConstView<word> &src,
    const DvConstView<word> &p_prod) const {
  const NPInfo np = param_.LevelToNP(level_, 0);
  const int num_q = np.GetNumQ();
  const int n = param_.degree_;
  AssertTrue(src.TotalSize() == num_q * n, "PseudoModUp src size mismatch");
  AssertTrue(dst.TotalSize() == num_q * n, "PseudoModUp dst size mismatch");
  AssertTrue(p_prod.TotalSize() == num_q, "PseudoModUp p_prod size mismatch");
  chd_limb_map m = NoSkipMap(param_, np);
  chd_accum_src s = {};
  s.src[0] = src.data();
  s.common = p_prod.data();
  word *d = dst.data();
  K(chd_k_cpaccum(&ntt_.Tables(), &m, &d, 1, nullptr, 0, &s, 1, 1, num_q,
                  CurrentStream()));
}

void ModSwitchHandler<uint32_t>::ModDown(DvView<word> &dst,
                                         const DvConstView<word> &src) const {
  const int n = param_.degree_;
  const NPInfo np = param_.LevelToNP(level_, num_aux_);
  AssertTrue(src.AuxSize() == np.num_aux_ * n &&
                 src.QSize() == np.GetNumQ() * n,
             "ModDown: src size mismatch");
  AssertTrue(dst.AuxSize() == 0 && dst.QSize() == np.GetNumQ() * n,
             "ModDown: dst size mismatch");
  ModDownWorker(dst, src, Kind::ModDown);
}

void ModSwitchHandler<uint32_t>::Rescale(DvView<word> &dst,
                                         const DvConstView<word> &src) const {
  const int n = param_.degree_;
  AssertTrue(level_ > 0, "Not enough q primes to rescale");
  const NPInfo np = param_.LevelToNP(level_);
  const NPInfo next = param_.LevelToNP(level_ - 1);
  AssertTrue(src.AuxSize() == 0 && src.QSize() == np.GetNumQ() * n,
             "Rescale: src size mismatch");
  AssertTrue(dst.AuxSize() == 0 && dst.QSize() == next.GetNumQ() * n,
             "Rescale: dst size mismatch");
  ModDownWorker(dst, src, Kind::Rescale);
}

void ModSwitchHandler<uint32_t>::ModDownAndRescale(
    DvView<word> &dst, const DvConstView<word> &src) const {
  const int n = param_.degree_;
  AssertTrue(level_ > 0, "Not enough q primes to rescale");
  const NPInfo np = param_.LevelToNP(level_, num_aux_);
  const NPInfo next = param_.LevelToNP(level_ - 1);
  AssertTrue(src.AuxSize() == np.num_aux_ * n &&
                 src.QSize() == np.GetNumQ() * n,
             "ModDownAndRescale: src size mismatch");
  AssertTrue(dst.AuxSize() == 0 && dst.QSize() == next.GetNumQ() * n,
             "ModDownAndRescale: dst size mismatch");
  ModDownWorker(dst, src, Kind::ModDownAndRescale);
}

// src/core/ModSwitch.cu:566-684 (kFuseModDownEpilogue)
void ModSwitchHandler<uint32_t>::ModDownWorker(DvView<word> &dst,
                                               const DvConstView<word> &src,
                                               Kind kind) const {
  ModDownMulti({dst.data()}, src.data(), 0, kind);
}

// ModDownWorker over num_polys polynomials with one launch per phase:
// INTTForModDown (centre), BConv, NTTForModDown.
bool ModSwitchHandler<uint32_t>::ModDownInttRange(Kind kind, int *first,
                                                  int *count) const {
  if (kind == Kind::Rescale || (kind != Kind::ModDown && level_ == 0))
    return false;
  const NPInfo np_src = param_.LevelToNP(level_, num_aux_);
  const NPInfo np_dst =
      param_.LevelToNP(kind == Kind::ModDown ? level_ : level_ - 1, 0);
  const NPInfo np_non_intt(std::min(np_src.num_main_, np_dst.num_main_),
                           std::min(np_src.num_ter_, np_dst.num_ter_), 0);
  if (np_src.num_ter_ > np_non_intt.num_ter_) return false;  // ter limbs
  *first = np_src.num_ter_ + np_non_intt.num_main_;
  *count = np_src.GetNumTotal() - np_non_intt.GetNumTotal();
  return true;
}

void ModSwitchHandler<uint32_t>::ModDownShape(Kind kind, NPInfo *np_src,
                                              NPInfo *np_dst,
                                              NPInfo *np_non_intt) const {
  const int num_src_aux = kind == Kind::Rescale ? 0 : num_aux_;
  *np_src = param_.LevelToNP(level_, num_src_aux);
  *np_dst = param_.LevelToNP(kind == Kind::ModDown ? level_ : level_ - 1, 0);
  *np_non_intt = NPInfo(std::min(np_src->num_main_, np_dst->num_main_),
                        std::min(np_src->num_ter_, np_dst->num_ter_), 0);
}

size_t ModSwitchHandler<uint32_t>::ModDownScratchWords(
    Kind kind, int num_polys, bool intt_rows_given) const {
  NPInfo np_src, np_dst, np_non_intt;
  ModDownShape(kind, &np_src, &np_dst, &np_non_intt);
  const size_t n = param_.degree_;
  const size_t src_len = np_src.GetNumTotal() - np_non_intt.GetNumTotal();
  const size_t dst_len = np_dst.GetNumTotal();
  // ModDownMulti's INTT output (unless given) and BConv output
  return (intt_rows_given ? 0 : num_polys * src_len * n) +
         num_polys * dst_len * n;
}

void ModSwitchHandler<uint32_t>::ModDownMulti(const std::vector<word *> &dst,
                                              const word *src,
                                              long long src_pstride,
                                              Kind kind,
                                              word *intt_rows) const {
  const int n = param_.degree_;
  const int num_polys = static_cast<int>(dst.size());
  AssertTrue(num_polys >= 1 && num_polys <= CHD_MAX_JOBS,
             "ModDown: 1 to CHD_MAX_JOBS polynomials per call");
  AssertTrue(kind == Kind::ModDown || level_ > 0,
             "Not enough q primes to rescale");
  NPInfo np_src, np_dst, np_non_intt;
  ModDownShape(kind, &np_src, &np_dst, &np_non_intt);
  const int src_len = np_src.GetNumTotal() - np_non_intt.GetNumTotal();
  const int dst_len = np_dst.GetNumTotal();
  const SwitchTable &st = kind == Kind::ModDown   ? mod_down_
                          : kind == Kind::Rescale ? rescale_
                                                  : mod_down_rescale_;
  AssertTrue(st.src_len == src_len && st.dst_len == dst_len,
             "ModDown: constant table mismatch");
  const long long ilen = static_cast<long long>(src_len) * n;
  Workspace::Use use_ws(ws_);
  Scratch intt_buf(ws_, intt_rows ? 0 : static_cast<size_t>(num_polys) * ilen);
  word *const intt = intt_rows ? intt_rows : intt_buf.data();
  for (int p = 0; p < num_polys; p++) {
    AssertTrue(dst[p] != nullptr, "ModDown: null destination");
    // INTTForModDown requires src != dst per polynomial (the polynomials
    // of src may lie in separate allocations, src_pstride of either sign)
    AssertTrue(reinterpret_cast<uintptr_t>(dst[p]) !=
                   reinterpret_cast<uintptr_t>(src) +
                       static_cast<uintptr_t>(4LL * p * src_pstride),
               "ModDown: src and dst should be different");
  }
  // NTTForModDown's epilogue operand src2 (the kept limbs of the source) is
  // read while other workgroups write the destinations, and with few
  // destination limbs the BConv writes them before that: no destination
  // may overlap any polynomial's src2, checked before anything is launched
  const int src2_off = std::max(0, np_src.num_ter_ - np_dst.num_ter_);
  const int s2_lo = np_dst.num_ter_ - np_non_intt.num_ter_;
  const int s2_hi = s2_lo + np_non_intt.GetNumQ();
  if (s2_hi > s2_lo)
    for (int p = 0; p < num_polys; p++)
      AssertTrue(chd::sets_disjoint_words(
                     src + static_cast<size_t>(src2_off) * n, src_pstride,
                     num_polys, static_cast<long long>(s2_hi - s2_lo) * n,
                     dst[p], 0, 1, static_cast<long long>(dst_len) * n),
                 "ModDown: the kept source limbs overlap a destination");
  // INTTForModDown (NTT.cu:973-1128) of all polynomials: either the top
  // main limbs (case 1) or the leading terminal limbs (case 2), then the
  // aux limbs when the source has them
  const bool intt_on_main = np_src.num_main_ > np_non_intt.num_main_;
  const bool intt_on_ter = np_src.num_ter_ > np_non_intt.num_ter_;
  AssertTrue(!intt_on_main || !intt_on_ter,
             "INTTForModDown: Invalid np combination");
  chd_limb_map mi{};
  mi.skip_lo = INT_MAX;
  size_t off = 0;
  if (!intt_on_ter) {
    mi.num_q = np_src.num_main_ - np_non_intt.num_main_;
    mi.tab_off = param_.GetMaxNumTer() + np_non_intt.num_main_;
    mi.tab_gap = param_.MainLeft(np_src);
    off = static_cast<size_t>(np_src.num_ter_ + np_non_intt.num_main_) * n;
  } else {
    mi.num_q = np_src.num_ter_ - np_non_intt.num_ter_;
    mi.tab_off = param_.TerLeft(np_src);
    mi.tab_gap = param_.GetMaxNumMain() + np_non_intt.num_ter_;
    mi.src_gap = np_src.GetNumQ() - mi.num_q;
  }
  if (intt_rows != nullptr) {
    // the first pass was done by the key accumulation (ModDownInttRange)
    AssertTrue(!intt_on_ter, "ModDown: fused INTT needs main INTT limbs");
    K(chd_k_ntt_inv_cols(&ntt_.Tables(), &mi, intt, ilen, src_len, num_polys,
                         st.const1.data(), 1, CurrentStream()));
  } else {
    K(chd_k_ntt_inv(&ntt_.Tables(), &mi, intt, ilen, src + off, src_pstride,
                    src_len, num_polys, st.const1.data(), 1, CurrentStream()));
  }
  chd_limb_map m = NoSkipMap(param_, np_dst);
  const DeviceVector<word> &ipp =
      kind == Kind::ModDown   ? inv_prime_prod_
      : kind == Kind::Rescale ? rescale_inv_prime_prod_
                              : mod_down_rescale_inv_prime_prod_;
  // BitPacker padding of the kept limbs when primes are restored; with an
  // empty restore range it is ToMont(1), the identity on the canonical src2
  // limbs, and the multiply is skipped (nullptr)
  const DeviceVector<word> &padv = kind == Kind::Rescale
                                       ? rescale_padding_
                                       : mod_down_rescale_padding_;
  const word *pad =
      kind != Kind::ModDown && padv.size() != 0 ? padv.data() : nullptr;
  // NTTForModDown (NTT.cu:417-604) with src2 = the untouched low limbs
  // (src2_off, s2_lo, s2_hi above). Few destination limbs: the single-pass NTT's time is one workgroup's
  // latency (~15 us whatever the limb count), so the BConv writes the
  // destination and the two-pass NTT runs in place on it, its passes
  // spread over many small workgroups (HMult at L = 4, 8, 12, 16: 6.4, 5.8,
  // 3.2 and 2.2 us faster; at 38 and 46 limbs the single pass is ahead)
  const bool one_src =
      st.src_len == 1 && st.bconv1.size() == static_cast<size_t>(dst_len);
  const bool few = num_polys * dst_len <= (one_src ? CHD_SMALL_RESCALE_LIMBS
                                                   : CHD_SMALL_MODDOWN_LIMBS);
  if (!few && one_src) {
    // one source (Rescale): the NTT forms each limb's BConv, the source
    // times that limb's table entry, from the one INTT limb as it reads it
    K(chd_k_ntt_fwd_moddown_bconv1_multi(
        &ntt_.Tables(), &m, dst.data(), num_polys, dst_len,
        reinterpret_cast<const int32_t *>(intt), ilen, st.bconv1.data(),
        src + static_cast<size_t>(src2_off) * n, src_pstride, s2_lo, s2_hi,
        ipp.data(), pad, CurrentStream()));
    return;
  }
  chd_bconv_job jobs[CHD_MAX_JOBS] = {};
  for (int p = 0; p < num_polys; p++) {
    jobs[p].dst = dst[p];
    jobs[p].src = reinterpret_cast<const int32_t *>(intt) + p * ilen;
    jobs[p].table = st.table.as<void>();
    jobs[p].src_len = src_len;
    jobs[p].dst_len = dst_len;
    jobs[p].skip_lo = INT_MAX;
    jobs[p].skip_len = 0;
  }
  if (few) {
    K(chd_k_bconv_batch(&ntt_.Tables(), &m, jobs, num_polys,
                        CurrentStream()));
    K(chd_k_ntt_fwd_moddown_multi(&ntt_.Tables(), &m, dst.data(), num_polys,
                                  dst_len, nullptr, 0,
                                  src + static_cast<size_t>(src2_off) * n,
                                  src_pstride, s2_lo, s2_hi, ipp.data(), pad,
                                  CurrentStream()));
    return;
  }
  // BConv into a temporary so that the NTT below reads it and writes dst in
  // one pass (the single-pass forward NTT cannot run in place)
  Scratch conv(ws_, static_cast<size_t>(num_polys) * dst_len * n);
  for (int p = 0; p < num_polys; p++)
    jobs[p].dst = conv.data() + static_cast<size_t>(p) * dst_len * n;
  K(chd_k_bconv_batch(&ntt_.Tables(), &m, jobs, num_polys, CurrentStream()));
  K(chd_k_ntt_fwd_moddown_multi(&ntt_.Tables(), &m, dst.data(), num_polys,
                                dst_len, conv.data(),
                                static_cast<long long>(dst_len) * n,
                                src + static_cast<size_t>(src2_off) * n,
                                src_pstride, s2_lo, s2_hi, ipp.data(), pad,
                                CurrentStream()));
}

// ---------------------------------------------------------------- Context --
std::shared_ptr<Context<uint32_t>> Context<uint32_t>::Create(
    const Parameter<word> &param) {
  return std::shared_ptr<Context<word>>(new Context<word>(param));
}

// src/core/Context.cpp:68-124
Context<uint32_t>::Context(const Parameter<word> &param)
    : param_(param),
      elem_handler_(param, ntt_handler_),
      ntt_handler_(param),
      encoder_(param, ntt_handler_) {
  // the reference's MemoryPool member (Context.h:84): this parameter set's
  // bins in the device pool every DeviceVector draws from
  MemoryPool::Current().AddBins(static_cast<size_t>(param_.degree_) *
                                    sizeof(word),
                                param_.alpha_, param_.L_);
  Ciphertext<word>::SetDegree(param_.degree_);
  {
    // arena for the largest call at the top level: HMult holds the tensor
    // (3 Lq), the accumulator (2 T) and ModUp's groups plus its INTT
    // (beta T + Lq); ModDown's INTT (at most 2 (alpha + 2) limbs) and BConv
    // output (2 Lq) and HRot's permute input (2 Lq) fit in what the ModUp
    // part leaves
    const NPInfo top = param_.LevelToNP(param_.max_level_);
    const size_t lq = top.GetNumQ();
    const size_t t = lq + param_.alpha_;
    const size_t beta = DivCeil(top.num_main_ + param_.GetMaxNumTer(),
                                param_.alpha_);
    const size_t moddown = 2 * (param_.alpha_ + 2) + 2 * lq;
    const size_t hmult =
        3 * lq + 2 * t + std::max(beta * t + lq, moddown + 2 * lq);
    // the hoisted giant step holds three extended pairs and a ModDown
    // output while a key switch runs (Hoist.cu:939-957)
    const size_t hoist = 6 * t + lq + beta * t + lq + moddown;
    const size_t limbs = std::max(hmult, hoist);
    ws_.reset(new Workspace(limbs * param_.degree_));
  }
  mod_switch_handlers_.reserve(param_.max_level_ + 1);
  for (int level = 0; level <= param_.max_level_; level++)
    mod_switch_handlers_.emplace_back(param_, level, elem_handler_,
                                      ntt_handler_, ws_.get());
  const NPInfo np = param_.LevelToNP(param_.max_level_, param_.alpha_);
  const std::vector<word> primes = param_.GetPrimeVector(np);
  const int num_q = np.GetNumQ();
  std::vector<word> h(num_q, 1);
  for (int i = 0; i < num_q; i++) {
    for (int j = 0; j < np.num_aux_; j++)
      h[i] = pm::mulmod(h[i], primes[num_q + j], primes[i]);
    h[i] = pm::to_mont(h[i], primes[i]);
  }
  p_prod_.resize(num_q);
  HipCheck(hipMemcpy(p_prod_.data(), h.data(), num_q * sizeof(word),
                     hipMemcpyHostToDevice),
           "hipMemcpy");
  // level-down constants: EncodeConstant(1.0) at each level's default scale
  // (Context.cpp:102-107; there only built with sparse-secret
  // encapsulation, here always, so LevelDown works for every parameter set)
  level_down_consts_.resize(param_.default_encryption_level_ + 1);
  for (int i = param_.default_encryption_level_; i > 0; i--)
    encoder_.EncodeConstant(level_down_consts_[i], i, param_.GetScale(i), 1.0);
}

DvConstView<uint32_t> Context<uint32_t>::GetPProd(const NPInfo &np) const {
  return DvConstView<word>(p_prod_.data() + param_.TerLeft(np), np.GetNumQ(),
                           0);
}

void Context<uint32_t>::TensorV(int level, CtRef res, CtCRef a,
                                CtCRef b) const {
  const NPInfo np = param_.LevelToNP(level);
  const int sz = np.GetNumQ() * param_.degree_;
  std::vector<DvView<word>> d{DvView<word>(res.bx, sz, 0),
                              DvView<word>(res.ax, sz, 0),
                              DvView<word>(res.rx, sz, 0)};
  elem_handler_.Tensor(d, np,
                       {DvConstView<word>(a.bx, sz, 0),
                        DvConstView<word>(a.ax, sz, 0)},
                       {DvConstView<word>(b.bx, sz, 0),
                        DvConstView<word>(b.ax, sz, 0)});
}

// src/core/Context.cpp:609-712: ModUp, PAccum over the dnum groups and
// CAccum, fused. ModUpGroups leaves every group after its column pass; one
// kernel then finishes the NTT of each group limb by limb, multiplies by the
// key and accumulates, so the ModUp output is written and read once.
void Context<uint32_t>::KeyMultNoModDownV(int level, word *acc_b, word *acc_a,
                                          const word *d, const word *cb,
                                          const word *ca,
                                          const EvkRef &key) const {
  KeyAccumulate(level, acc_b, acc_a, d, cb, ca, nullptr, nullptr, key);
}

void Context<uint32_t>::KeyMultTensorV(int level, word *acc_b, word *acc_a,
                                       CtCRef a, CtCRef b,
                                       const EvkRef &key) const {
  KeyAccumulate(level, acc_b, acc_a, nullptr, nullptr, nullptr, &a, &b, key);
}

// KeyAccumulate followed by ModDown (or ModDownAndRescale) into res, with
// ModDown's first INTT pass done by the key accumulation when the INTT limbs
// are contiguous (no terminal limb dropped); the accumulator limbs that the
// INTT covers are then never stored.
void Context<uint32_t>::KeySwitchDown(int level, CtRef res, const word *d,
                                      const word *cb, const word *ca,
                                      const CtCRef *ta, const CtCRef *tb,
                                      const EvkRef &key, bool rescale) const {
  const int n = param_.degree_;
  const int num_q = param_.LevelToNP(level).GetNumQ();
  const int total = num_q + param_.alpha_;
  const auto kind = rescale ? ModSwitchHandler<word>::Kind::ModDownAndRescale
                            : ModSwitchHandler<word>::Kind::ModDown;
  const auto &ms = mod_switch_handlers_.at(level);
  int first = 0, count = 0;
  const bool fused = ms.ModDownInttRange(kind, &first, &count);
  Workspace::Use use_ws(ws_.get());
  Scratch acc(ws_.get(), static_cast<size_t>(2) * total * n);
  Scratch rows(ws_.get(), fused ? static_cast<size_t>(2) * count * n : 0);
  word *acc_b = acc.data();
  word *acc_a = acc.data() + static_cast<size_t>(total) * n;
  word *rows_b = fused ? rows.data() : nullptr;
  word *rows_a = fused ? rows.data() + static_cast<size_t>(count) * n : nullptr;
  KeyAccumulate(level, acc_b, acc_a, d, cb, ca, ta, tb, key, nullptr, rows_b,
                rows_a, first);
  ms.ModDownMulti({res.bx, res.ax}, acc_b, static_cast<long long>(total) * n,
                  kind, rows_b);
}

size_t Context<uint32_t>::KeySwitchScratchWords(int level,
                                                bool rescale) const {
  // KeySwitchDown: accumulator and ModDown's first INTT pass for the whole
  // call, then KeyAccumulate's ModUp groups and INTT or ModDownMulti's
  // temporaries, one after the other
  const size_t n = param_.degree_;
  const size_t num_q = param_.LevelToNP(level).GetNumQ();
  const size_t total = num_q + param_.alpha_;
  const auto kind = rescale ? ModSwitchHandler<word>::Kind::ModDownAndRescale
                            : ModSwitchHandler<word>::Kind::ModDown;
  const auto &ms = mod_switch_handlers_.at(level);
  int first = 0, count = 0;
  const bool fused = ms.ModDownInttRange(kind, &first, &count);
  const size_t acc = 2 * total * n + (fused ? 2 * count * n : 0);
  const size_t modup = ms.NumGroups() * total * n + num_q * n;
  return acc + std::max(modup, ms.ModDownScratchWords(kind, 2, fused));
}

void Context<uint32_t>::KeyMultExtV(int level, word *acc_b, word *acc_a,
                                    const word *d, const word *add_b,
                                    const EvkRef &key) const {
  KeyAccumulate(level, acc_b, acc_a, d, nullptr, nullptr, nullptr, nullptr,
                key, add_b);
}

// src/core/Context.cpp:609-643 on views: the PAccum of the non-empty dnum
// groups of a caller-held ModUp with the key read from the level's first
// chain position (the key's extra_ view, Context.cpp:640)
void Context<uint32_t>::KeyMultModUpV(int level, word *acc_b, word *acc_a,
                                      const word *const *modup,
                                      const EvkRef &key) const {
  const NPInfo a_np = param_.LevelToNP(level);
  const int n = param_.degree_;
  const int num_q = a_np.GetNumQ();
  const int num_aux = key.np.num_aux_;
  AssertTrue(num_aux == param_.alpha_, "Invalid setting for MultKeyNoModDown");
  const int prime_offset = param_.GetMaxNumTer() - a_np.num_ter_;
  const int padded_num_q = num_q + prime_offset;
  const int beta = DivCeil(padded_num_q, num_aux);
  AssertTrue(static_cast<int>(key.bx.size()) >= beta &&
                 key.bx.size() == key.ax.size(),
             "Beta mismatch");
  const int key_q = key.np.GetNumQ() - prime_offset;
  AssertTrue(key_q >= num_q, "MultKeyNoModDown: key level below input level");
  const NPInfo np(a_np.num_main_, a_np.num_ter_, num_aux);
  const int total = np.GetNumTotal() * n;
  const int aux_words = num_aux * n;
  std::vector<std::vector<DvConstView<word>>> key_views;
  std::vector<DvConstView<word>> modup_views;
  for (int i = 0; i < beta; i++) {
    if (std::min((i + 1) * num_aux, padded_num_q) <= prime_offset) continue;
    AssertTrue(modup[i] != nullptr, "MultKeyNoModDown: null ModUp group");
    const int key_words = (key_q + num_aux) * n;
    key_views.push_back(
        {DvConstView<word>(key.bx[i] + static_cast<size_t>(prime_offset) * n,
                           key_words, aux_words),
         DvConstView<word>(key.ax[i] + static_cast<size_t>(prime_offset) * n,
                           key_words, aux_words)});
    modup_views.emplace_back(modup[i], total, aux_words);
  }
  std::vector<DvView<word>> acc{DvView<word>(acc_b, total, aux_words),
                                DvView<word>(acc_a, total, aux_words)};
  elem_handler_.PAccum(acc, np, key_views, modup_views);
}

// src/core/Context.cpp:609-643
void Context<uint32_t>::MultKeyNoModDown(Ct &accum,
                                         const std::vector<Dv> &a_modup,
                                         const Ct &a_orig,
                                         const Evk &key) const {
  const NPInfo a_np = a_orig.GetNP();
  const int level = param_.NPToLevel(a_np);
  AssertTrue(key.GetNP().num_aux_ == param_.alpha_,
             "Invalid setting for MultKeyNoModDown");
  AssertTrue(&accum != &a_orig,
             "In-place operation is not supported for MultKeyNoModDown");
  const int num_aux = param_.alpha_;
  const int prime_offset = param_.GetMaxNumTer() - a_np.num_ter_;
  const int padded_num_q = a_np.GetNumQ() + prime_offset;
  const int beta = DivCeil(padded_num_q, num_aux);
  AssertTrue(key.GetBeta() >= beta && static_cast<int>(a_modup.size()) == beta,
             "Beta mismatch");
  const NPInfo np(a_np.num_main_, a_np.num_ter_, num_aux);
  const size_t total = static_cast<size_t>(np.GetNumTotal()) * param_.degree_;
  std::vector<const word *> modup(beta, nullptr);
  for (int i = 0; i < beta; i++) {
    if (std::min((i + 1) * num_aux, padded_num_q) <= prime_offset) continue;
    AssertTrue(a_modup[i].size() == total,
               "MultKeyNoModDown: ModUp group size mismatch");
    modup[i] = a_modup[i].data();
  }
  const double scale = a_orig.GetScale();
  const int slots = a_orig.GetNumSlots();
  accum.RemoveRx();
  accum.ModifyNP(np);
  accum.SetScale(scale);
  accum.SetNumSlots(slots);
  KeyMultModUpV(level, accum.bx_.data(), accum.ax_.data(), modup.data(),
                RefOfKey(key));
}

// src/core/Context.cpp:645-712: ModUp, PAccum and CAccum in the fused key
// accumulation (one launch after the ModUp's INTT, BConv and column pass)
void Context<uint32_t>::MultKeyNoModDown(Ct &accum, const Ct &a,
                                         const Evk &key) const {
  const NPInfo a_np = a.GetNP();
  AssertTrue(a_np.num_aux_ == 0,
             "MultKeyNoModDown is not supported for ciphertexts with p "
             "primes");
  AssertTrue(&accum != &a,
             "In-place operation is not supported for MultKeyNoModDown");
  const int level = param_.NPToLevel(a_np);
  AssertTrue(key.GetNP().num_aux_ == param_.alpha_,
             "Invalid setting for MultKeyNoModDown");
  const double scale = a.GetScale();
  const int slots = a.GetNumSlots();
  accum.RemoveRx();
  accum.ModifyNP(NPInfo(a_np.num_main_, a_np.num_ter_, param_.alpha_));
  accum.SetScale(scale);
  accum.SetNumSlots(slots);
  const EvkRef k = RefOfKey(key);
  if (a.HasRx())  // relinearisation: ModUp(rx), p_prod * (bx, ax)
    KeyMultNoModDownV(level, accum.bx_.data(), accum.ax_.data(),
                      a.rx_.data(), a.bx_.data(), a.ax_.data(), k);
  else  // MultKey: ModUp(ax), p_prod * bx
    KeyMultNoModDownV(level, accum.bx_.data(), accum.ax_.data(),
                      a.ax_.data(), a.bx_.data(), nullptr, k);
}

void Context<uint32_t>::KeyAccumulate(int level, word *acc_b, word *acc_a,
                                      const word *d, const word *cb,
                                      const word *ca, const CtCRef *ta,
                                      const CtCRef *tb, const EvkRef &key,
                                      const word *add_b, word *intt_b,
                                      word *intt_a, int intt_lo) const {
  const NPInfo a_np = param_.LevelToNP(level);
  const int n = param_.degree_;
  const int num_q = a_np.GetNumQ();
  const int num_aux = key.np.num_aux_;
  AssertTrue(num_aux == param_.alpha_, "Invalid setting for MultKeyNoModDown");
  const int prime_offset = param_.GetMaxNumTer() - a_np.num_ter_;
  const int beta = DivCeil(num_q + prime_offset, num_aux);
  AssertTrue(static_cast<int>(key.bx.size()) >= beta &&
                 key.bx.size() == key.ax.size(),
             "Beta mismatch");
  const auto &ms = mod_switch_handlers_.at(level);
  AssertTrue(ms.GetBeta() == beta, "MultKeyNoModDown: beta mismatch");
  // the groups before ms.FirstGroup() hold no limb of this level and are
  // skipped with their keys (Context.cpp:637-642)
  const int groups = ms.NumGroups();
  const int first = ms.FirstGroup();
  AssertTrue(groups <= CHD_MAX_JOBS, "MultKeyNoModDown: dnum too large");
  const int total = num_q + num_aux;
  const long long gs = static_cast<long long>(total) * n;
  Workspace::Use use_ws(ws_.get());
  Scratch buf(ws_.get(),
              static_cast<size_t>(groups) * gs + static_cast<size_t>(num_q) * n);
  const bool tensor = ta != nullptr;
  ms.ModUpGroups(buf.data(), gs,
                 DvConstView<word>(tensor ? ta->ax : d, num_q * n, 0),
                 buf.data() + groups * gs, false, tensor ? tb->ax : nullptr);
  chd_keyacc_args k{};
  k.num_q = num_q;
  k.tab_off = param_.TerLeft(a_np);
  k.tab_gap = param_.MainLeft(a_np);
  k.alpha = num_aux;
  k.beta = groups;
  k.group_shift = ms.GroupShift();
  k.modup = buf.data();
  k.group_stride = gs;
  k.d = d;
  for (int z = 0; z < groups; z++) {
    k.kb[z] = key.bx[first + z] + static_cast<size_t>(prime_offset) * n;
    k.ka[z] = key.ax[first + z] + static_cast<size_t>(prime_offset) * n;
  }
  // key layout: q limbs of the key's level, then its aux limbs
  k.key_gap = static_cast<long long>(key.np.GetNumQ() - prime_offset - num_q) * n;
  AssertTrue(k.key_gap >= 0, "MultKeyNoModDown: key level below input level");
  k.p_prod = GetPProd(a_np).data();
  k.cb = cb;
  k.ca = ca;
  k.acc_b = acc_b;
  k.acc_a = acc_a;
  k.add_b = add_b;
  k.intt_b = intt_b;
  k.intt_a = intt_a;
  k.intt_lo = intt_lo;
  if (tensor) {
    k.d = nullptr;
    k.cb = nullptr;
    k.ca = nullptr;
    k.b1 = ta->bx;
    k.a1 = ta->ax;
    k.b2 = tb->bx;
    k.a2 = tb->ax;
  }
  K(chd_k_modup_keyacc(&ntt_handler_.Tables(), &k, CurrentStream()));
}

void Context<uint32_t>::KeyMultExtBatchV(int level, int num,
                                         word *const *acc_b,
                                         word *const *acc_a, const word *d,
                                         long long d_stride,
                                         const word *add_b,
                                         long long add_stride,
                                         const EvkRef *const *keys) const {
  const NPInfo a_np = param_.LevelToNP(level);
  const int n = param_.degree_;
  const int num_q = a_np.GetNumQ();
  const int num_aux = param_.alpha_;
  AssertTrue(num >= 1 && num <= CHD_MAX_JOBS,
             "KeyMultExtBatch: 1 to CHD_MAX_JOBS inputs per batch");
  const int prime_offset = param_.GetMaxNumTer() - a_np.num_ter_;
  const int beta = DivCeil(num_q + prime_offset, num_aux);
  const auto &ms = mod_switch_handlers_.at(level);
  AssertTrue(ms.GetBeta() == beta, "MultKeyNoModDown: beta mismatch");
  const int groups = ms.NumGroups();
  const int first = ms.FirstGroup();
  AssertTrue(groups <= CHD_MAX_JOBS, "MultKeyNoModDown: dnum too large");
  const int total = num_q + num_aux;
  const long long gs = static_cast<long long>(total) * n;
  Workspace::Use use_ws(ws_.get());
  Scratch buf(ws_.get(), static_cast<size_t>(num) * groups * gs +
                             static_cast<size_t>(num) * num_q * n);
  ms.ModUpGroupsBatch(buf.data(), gs, d, d_stride, num,
                      buf.data() + static_cast<size_t>(num) * groups * gs);
  chd_keyacc_args jobs[CHD_MAX_JOBS] = {};
  for (int i = 0; i < num; i++) {
    const EvkRef &key = *keys[i];
    AssertTrue(key.np.num_aux_ == num_aux,
               "Invalid setting for MultKeyNoModDown");
    AssertTrue(static_cast<int>(key.bx.size()) >= beta &&
                   key.bx.size() == key.ax.size(),
               "Beta mismatch");
    chd_keyacc_args &k = jobs[i];
    k.num_q = num_q;
    k.tab_off = param_.TerLeft(a_np);
    k.tab_gap = param_.MainLeft(a_np);
    k.alpha = num_aux;
    k.beta = groups;
    k.group_shift = ms.GroupShift();
    k.modup = buf.data() + static_cast<size_t>(i) * groups * gs;
    k.group_stride = gs;
    k.d = d + i * d_stride;
    for (int z = 0; z < groups; z++) {
      k.kb[z] = key.bx[first + z] + static_cast<size_t>(prime_offset) * n;
      k.ka[z] = key.ax[first + z] + static_cast<size_t>(prime_offset) * n;
    }
    k.key_gap =
        static_cast<long long>(key.np.GetNumQ() - prime_offset - num_q) * n;
    AssertTrue(k.key_gap >= 0, "MultKeyNoModDown: key level below input level");
    k.p_prod = GetPProd(a_np).data();
    k.acc_b = acc_b[i];
    k.acc_a = acc_a[i];
    k.add_b = add_b + i * add_stride;
  }
  K(chd_k_modup_keyacc_batch(&ntt_handler_.Tables(), jobs, num,
                             CurrentStream()));
}

// src/core/Context.cpp:862-871 with 714-737 / 559-607
void Context<uint32_t>::HMultV(int level, CtRef res, CtCRef a, CtCRef b,
                               const EvkRef &key, bool rescale) const {
  AssertTrue(!rescale || level > 0, "Not enough q primes to rescale");
  // Tensor fused into ModUp's INTT and the key accumulation
  KeySwitchDown(level, res, nullptr, nullptr, nullptr, &a, &b, key, rescale);
}

// src/core/Context.cpp:739-774
void Context<uint32_t>::RescaleV(int level, CtRef res, CtCRef a) const {
  AssertTrue(level > 0, "Not enough q primes to rescale");
  const int n = param_.degree_;
  const int nq = param_.LevelToNP(level).GetNumQ();
  const int nq1 = param_.LevelToNP(level - 1).GetNumQ();
  const auto &ms = mod_switch_handlers_.at(level);
  if (res.bx != res.ax) {
    // bx and ax in one launch per phase (INTT of the top limb, BConv, NTT
    // with the rescale epilogue): polynomial 1 is addressed as a.bx + its
    // distance to a.ax, whatever the sign or size of that distance
    const long long stride =
        (static_cast<long long>(reinterpret_cast<intptr_t>(a.ax)) -
         static_cast<long long>(reinterpret_cast<intptr_t>(a.bx))) /
        static_cast<long long>(sizeof(word));
    ms.ModDownMulti({res.bx, res.ax}, a.bx, stride,
                    ModSwitchHandler<word>::Kind::Rescale);
  } else {
    DvView<word> db(res.bx, nq1 * n, 0), da(res.ax, nq1 * n, 0);
    ms.Rescale(db, DvConstView<word>(a.bx, nq * n, 0));
    ms.Rescale(da, DvConstView<word>(a.ax, nq * n, 0));
  }
  if (a.rx != nullptr && res.rx != nullptr) {
    DvView<word> dr(res.rx, nq1 * n, 0);
    ms.Rescale(dr, DvConstView<word>(a.rx, nq * n, 0));
  }
}

// src/core/Context.cpp:584-607
void Context<uint32_t>::MultKeyV(int level, CtRef res, CtCRef a,
                                 const EvkRef &key) const {
  KeySwitchDown(level, res, a.ax, a.bx, nullptr, nullptr, nullptr, key, false);
}

void Context<uint32_t>::PermuteV(int level, CtRef res, CtCRef a,
                                 int amount) const {
  const NPInfo np = param_.LevelToNP(level);
  const int sz = np.GetNumQ() * param_.degree_;
  std::vector<DvView<word>> d{DvView<word>(res.bx, sz, 0),
                              DvView<word>(res.ax, sz, 0)};
  elem_handler_.Permute(d, np, amount,
                        {DvConstView<word>(a.bx, sz, 0),
                         DvConstView<word>(a.ax, sz, 0)});
}

// ------------------------------------------- Ciphertext-level entry points
namespace {
Context<uint32_t>::EvkRef RefOf(const EvaluationKey<uint32_t> &k) {
  Context<uint32_t>::EvkRef r;
  r.np = k.GetNP();
  for (int g = 0; g < k.GetBeta(); g++) {
    r.bx.push_back(k.bx_[g].data());
    r.ax.push_back(k.ax_[g].data());
  }
  return r;
}
}  // namespace

void Context<uint32_t>::Mult(Ct &res, const Ct &a, const Ct &b) const {
  AssertTrue(a.GetNP() == b.GetNP(), "Mult: NP mismatch");
  AssertTrue(!a.HasRx() && !b.HasRx(),
             "Relinearization required before Mult Ct x Ct");
  const int level = param_.NPToLevel(a.GetNP());
  // Tensor reads a and b fully before res is resized only when res aliases
  // neither; otherwise go through a temporary
  Ct tmp(a.GetNP(), true);
  TensorV(level, {tmp.bx_.data(), tmp.ax_.data(), tmp.rx_.data()},
          {a.bx_.data(), a.ax_.data(), nullptr},
          {b.bx_.data(), b.ax_.data(), nullptr});
  tmp.SetNumSlots(std::max(a.GetNumSlots(), b.GetNumSlots()));
  tmp.SetScale(a.GetScale() * b.GetScale());
  res = std::move(tmp);
}

void Context<uint32_t>::Relinearize(Ct &res, const Ct &a,
                                    const Evk &key) const {
  AssertTrue(a.HasRx(), "Relinearize requires aux");
  const int level = param_.NPToLevel(a.GetNP());
  const int n = param_.degree_;
  const int num_q = a.GetNP().GetNumQ();
  const int total = num_q + param_.alpha_;
  Ct out(a.GetNP());
  Workspace::Use use_ws(ws_.get());
  Scratch acc(ws_.get(), static_cast<size_t>(2) * total * n);
  KeyMultNoModDownV(level, acc.data(), acc.data() + static_cast<size_t>(total) * n,
                    a.rx_.data(), a.bx_.data(), a.ax_.data(), RefOf(key));
  mod_switch_handlers_.at(level).ModDownMulti(
      {out.bx_.data(), out.ax_.data()}, acc.data(),
      static_cast<long long>(total) * n, ModSwitchHandler<word>::Kind::ModDown);
  out.SetScale(a.GetScale());
  out.SetNumSlots(a.GetNumSlots());
  res = std::move(out);
}

void Context<uint32_t>::RelinearizeRescale(Ct &res, const Ct &a,
                                           const Evk &key) const {
  AssertTrue(a.HasRx(), "RelinearizeRescale requires aux");
  const int level = param_.NPToLevel(a.GetNP());
  const int n = param_.degree_;
  const int num_q = a.GetNP().GetNumQ();
  const int total = num_q + param_.alpha_;
  Ct out(param_.LevelToNP(level - 1));
  Workspace::Use use_ws(ws_.get());
  Scratch acc(ws_.get(), static_cast<size_t>(2) * total * n);
  KeyMultNoModDownV(level, acc.data(), acc.data() + static_cast<size_t>(total) * n,
                    a.rx_.data(), a.bx_.data(), a.ax_.data(), RefOf(key));
  mod_switch_handlers_.at(level).ModDownMulti(
      {out.bx_.data(), out.ax_.data()}, acc.data(),
      static_cast<long long>(total) * n,
      ModSwitchHandler<word>::Kind::ModDownAndRescale);
  out.SetScale(a.GetScale() / param_.GetRescalePrimeProd(level));
  out.SetNumSlots(a.GetNumSlots());
  res = std::move(out);
}

// src/core/Context.cpp:862-871: Mult, then Relinearize or
// RelinearizeRescale; here one fused pass (the tensor is never stored)
void Context<uint32_t>::HMult(Ct &res, const Ct &a, const Ct &b,
                              const Evk &mult_key, bool rescale) const {
  AssertTrue(a.GetNP() == b.GetNP(), "Mult: NP mismatch");
  AssertTrue(!a.HasRx() && !b.HasRx(),
             "Relinearization required before Mult Ct x Ct");
  const int level = param_.NPToLevel(a.GetNP());
  AssertTrue(!rescale || level > 0, "Not enough q primes to rescale");
  Ct out(rescale ? param_.LevelToNP(level - 1) : a.GetNP());
  HMultV(level, {out.bx_.data(), out.ax_.data(), nullptr},
         {a.bx_.data(), a.ax_.data(), nullptr},
         {b.bx_.data(), b.ax_.data(), nullptr}, RefOf(mult_key), rescale);
  const double scale = a.GetScale() * b.GetScale();
  out.SetScale(rescale ? scale / param_.GetRescalePrimeProd(level) : scale);
  out.SetNumSlots(std::max(a.GetNumSlots(), b.GetNumSlots()));
  res = std::move(out);
}

void Context<uint32_t>::MultKey(Ct &res, const Ct &a, const Evk &key) const {
  const int level = param_.NPToLevel(a.GetNP());
  Ct out(a.GetNP());
  MultKeyV(level, {out.bx_.data(), out.ax_.data(), nullptr},
           {a.bx_.data(), a.ax_.data(), nullptr}, RefOf(key));
  out.SetScale(a.GetScale());
  out.SetNumSlots(a.GetNumSlots());
  res = std::move(out);
}

void Context<uint32_t>::Rescale(Ct &res, const Ct &a) const {
  AssertTrue(a.GetNP().num_aux_ == 0,
             "Rescale is not supported for ciphertexts with p primes");
  const int level = param_.NPToLevel(a.GetNP());
  AssertTrue(level > 0, "Not enough q primes to rescale");
  Ct out(param_.LevelToNP(level - 1), a.HasRx());
  RescaleV(level, {out.bx_.data(), out.ax_.data(),
                   a.HasRx() ? out.rx_.data() : nullptr},
           {a.bx_.data(), a.ax_.data(), a.HasRx() ? a.rx_.data() : nullptr});
  out.SetNumSlots(a.GetNumSlots());
  out.SetScale(a.GetScale() / param_.GetRescalePrimeProd(level));
  res = std::move(out);
}

void Context<uint32_t>::Permute(Ct &res, const Ct &a, int rot_dist) const {
  int slots = a.GetNumSlots();
  int r = rot_dist % slots;
  if (r < 0) r += slots;
  const int level = param_.NPToLevel(a.GetNP());
  Ct out(a.GetNP());
  if (r == 0) {
    const size_t bytes = a.bx_.size() * sizeof(word);
    HipCheck(hipMemcpyAsync(out.bx_.data(), a.bx_.data(), bytes,
                            hipMemcpyDeviceToDevice, CurrentStream()),
             "hipMemcpyAsync");
    HipCheck(hipMemcpyAsync(out.ax_.data(), a.ax_.data(), bytes,
                            hipMemcpyDeviceToDevice, CurrentStream()),
             "hipMemcpyAsync");
  } else {
    PermuteV(level, {out.bx_.data(), out.ax_.data(), nullptr},
             {a.bx_.data(), a.ax_.data(), nullptr}, r);
  }
  out.SetNumSlots(a.GetNumSlots());
  out.SetScale(a.GetScale());
  res = std::move(out);
}

// src/core/Context.cpp:776-791: key switch first, then permute
void Context<uint32_t>::HRot(Ct &res, const Ct &a, const Evk &rot_key,
                             int rot_dist) const {
  int slots = a.GetNumSlots();
  int r = rot_dist % slots;
  if (r < 0) r += slots;
  Ct tmp;
  if (r == 0) {
    Permute(res, a, 0);
    return;
  }
  MultKey(tmp, a, rot_key);
  Permute(res, tmp, r);
}

Context<uint32_t>::EvkRef Context<uint32_t>::RefOfKey(const Evk &k) {
  return RefOf(k);
}

// ---------------------------------------------------------- HoistHandler --
// src/core/EvkRequest.cpp:7-17
void EvkRequest::AddRequest(int rot_idx, int level) {
  AssertTrue(rot_idx >= 0, "Invalid rotation index");
  AssertTrue(level >= 0, "Invalid level");
  auto it = find(rot_idx);
  if (it == end())
    emplace(rot_idx, level);
  else if (it->second < level)
    it->second = level;
}

// Hoist.cu:131-145 (CompilePlaintexts) and 146-173 (the bs/gs swap)
HoistHandler<uint32_t>::PtMap HoistHandler<uint32_t>::EncodeMap(
    const Context<word> &context, const PlainHoistMap &hoist_map,
    int pt_level, double pt_scale, bool suppress_bs_swap) {
  AssertTrue(!hoist_map.empty(), "Hoist: hoist_map should not be empty");
  const int alpha = context.param_.alpha_;
  const Encoder<word> &enc = context.encoder_;
  struct Job {
    int g, b;
    const Message *msg;
    Message rotated;
  };
  std::vector<Job> jobs;
  if (hoist_map.size() == 1 && hoist_map.begin()->first == 0 &&
      !suppress_bs_swap) {
    // single giant step: baby step b becomes giant step b with baby step 0,
    // its message rotated right by b
    for (const auto &[b, msg] : hoist_map.begin()->second) {
      const size_t sz = msg.size();
      AssertTrue(sz > 0, "Hoist: empty message");
      Message rot(sz);
      for (size_t i = 0; i < sz; i++) rot[(i + b) % sz] = msg[i];
      jobs.push_back(Job{b, 0, nullptr, std::move(rot)});
    }
  } else {
    for (const auto &[g, bs_map] : hoist_map)
      for (const auto &[b, msg] : bs_map) jobs.push_back(Job{g, b, &msg, {}});
  }
  // the host halves (special IFFT and residues) of up to `width` plaintexts
  // run on as many threads, then their uploads and NTTs in order
  const size_t width = std::max<size_t>(
      1, std::min<size_t>(16, std::thread::hardware_concurrency()));
  PtMap out;
  std::vector<std::vector<word>> mx(width);
  std::vector<int> slots(width);
  std::vector<std::exception_ptr> err(width);
  for (size_t start = 0; start < jobs.size(); start += width) {
    const size_t count = std::min(width, jobs.size() - start);
    auto host_half = [&](size_t k) {
      try {
        const Job &j = jobs[start + k];
        std::vector<Complex> padded =
            Encoder<word>::PadToPowerOfTwo(j.msg ? *j.msg : j.rotated);
        slots[k] = static_cast<int>(padded.size());
        mx[k] = enc.CoefficientResidues(pt_level, pt_scale, std::move(padded),
                                        alpha);
      } catch (...) {
        err[k] = std::current_exception();
      }
    };
    std::vector<std::thread> threads;
    for (size_t k = 1; k < count; k++) threads.emplace_back(host_half, k);
    host_half(0);
    for (std::thread &t : threads) t.join();
    for (size_t k = 0; k < count; k++)
      if (err[k]) std::rethrow_exception(err[k]);
    for (size_t k = 0; k < count; k++) {
      const Job &j = jobs[start + k];
      Pt &pt = out[j.g].try_emplace(j.b, NPInfo(0, 0, 0)).first->second;
      enc.EncodeResidues(pt, pt_level, pt_scale, slots[k], mx[k], alpha);
    }
  }
  return out;
}

HoistHandler<uint32_t>::HoistHandler(ConstContextPtr<word> context,
                                     const PlainHoistMap &hoist_map,
                                     int pt_level, double pt_scale,
                                     bool suppress_bs_swap)
    : HoistHandler(context,
                   EncodeMap(*context, hoist_map, pt_level, pt_scale,
                             suppress_bs_swap),
                   pt_level, pt_scale) {}

HoistHandler<uint32_t>::HoistHandler(ConstContextPtr<word> context,
                                     PtMap &&encoded, int pt_level,
                                     double pt_scale)
    : pt_level_(pt_level), pt_scale_(pt_scale), pt_map_(std::move(encoded)) {
  AssertTrue(!pt_map_.empty(), "Hoist: hoist_map should not be empty");
  const Parameter<word> &param = context->param_;
  const int n = param.degree_;
  const NPInfo np = param.LevelToNP(pt_level_, param.alpha_);
  bool only_bs0 = true;
  for (const auto &[gs, bs_map] : pt_map_) {
    AssertTrue(!bs_map.empty(), "Hoist: empty baby-step map");
    AssertTrue(gs >= 0 && gs < n / 2, "Hoist: invalid giant step");
    for (const auto &[bs, pt] : bs_map) {
      AssertTrue(bs >= 0 && bs < n / 2, "Hoist: invalid baby step");
      AssertTrue(pt.GetNP() == np && pt.mx_.size() ==
                     static_cast<size_t>(np.GetNumTotal()) * n,
                 "Hoist: plaintexts must hold pt_level's q primes and alpha "
                 "aux primes");
      only_bs0 = only_bs0 && bs == 0;
    }
  }
  if (only_bs0) {
    // giant steps with baby step 0 only: one giant step 0 whose baby steps
    // are the rotations, plaintexts permuted ahead (see the class comment)
    PtMap conv;
    std::map<int, Pt> &row = conv[0];
    const int aux_words = param.alpha_ * n;
    for (auto &[g, bs_map] : pt_map_) {
      Pt &src = bs_map.begin()->second;
      if (g == 0) {
        row.emplace(0, std::move(src));
        continue;
      }
      Pt dst(np, n);
      dst.SetScale(src.GetScale());
      dst.SetNumSlots(src.GetNumSlots());
      std::vector<DvView<word>> d = {dst.mx_.View(aux_words)};
      context->elem_handler_.Permute(d, np, g, {src.mx_.ConstView(aux_words)});
      row.emplace(g, std::move(dst));
    }
    HipCheck(hipStreamSynchronize(CurrentStream()), "hipStreamSynchronize");
    pt_map_ = std::move(conv);
    gs_only_ = pt_map_.at(0).size() > 1 || pt_map_.at(0).count(0) == 0;
  }
  for (const auto &[gs, bs_map] : pt_map_) {
    gs_indices_.push_back(gs);
    for (const auto &[bs, pt] : bs_map) bs_indices_.insert(bs);
  }
  AssertTrue(gs_indices_.size() == 1 || gs_indices_.front() == 0,
             "Hoist: a giant step 0 is required with several giant steps");
  AssertTrue(bs_indices_.size() <= 64, "Hoist: too many baby steps");
  const int num_gs = static_cast<int>(gs_indices_.size());
  if (num_gs > CHD_GS_MAX_GS && num_gs <= CHD_GS_WIDE_GS &&
      bs_indices_.size() <= CHD_GS_MAX_BS) {
    for (int w : {16, 24, 28, 32})
      if (wide_gs_ == 0 && num_gs <= w) wide_gs_ = w;
    const size_t pt_words = static_cast<size_t>(np.GetNumTotal()) * n;
    zero_pt_.Resize(pt_words * sizeof(word));
    HipCheck(hipMemset(zero_pt_.as<void>(), 0, pt_words * sizeof(word)),
             "hipMemset");
    if (wide_gs_ > num_gs) dummy_out_.Resize(2 * pt_words * sizeof(word));
    // baby steps in fours: padding columns (and the padding baby steps
    // themselves, at run time) are the zero plaintext
    wide_bs_ = (static_cast<int>(bs_indices_.size()) + 3) / 4 * 4;
    std::vector<const word *> table;
    table.reserve(static_cast<size_t>(wide_gs_) * wide_bs_);
    for (int k = 0; k < wide_gs_; k++) {
      const std::map<int, Pt> *pmap =
          k < num_gs ? &pt_map_.at(gs_indices_[k]) : nullptr;
      int j = 0;
      for (int b : bs_indices_) {
        const word *p = zero_pt_.as<const word>();
        if (pmap != nullptr) {
          auto it = pmap->find(b);
          if (it != pmap->end()) p = it->second.mx_.data();
        }
        table.push_back(p);
        j++;
      }
      for (; j < wide_bs_; j++) table.push_back(zero_pt_.as<const word>());
    }
    pt_table_.Upload(table);
#if CHD_GS_TILED
    // the real giant steps' plaintexts move into one tiled array, so that
    // each accumulation workgroup streams one contiguous run (one block of
    // one limb, every pair) instead of 1 KiB from each pair's allocation;
    // the per-pair copies are then given back (to the memory pool) and the
    // table points only at the zero plaintext: the wide accumulation reads
    // the tiled array, MinKS takes rows back out of it
    tiled_rows_ = num_gs;
    pt_tiled_.Resize(static_cast<size_t>(tiled_rows_) * wide_bs_ * pt_words *
                     sizeof(word));
    K(chd_k_gs_pack_tiled(pt_table_.as<const word *>(), tiled_rows_,
                          wide_bs_, np.GetNumTotal(), pt_tiled_.as<word>(),
                          CurrentStream()));
    HipCheck(hipStreamSynchronize(CurrentStream()), "hipStreamSynchronize");
    for (auto &[g, bs_map] : pt_map_)
      for (auto &[b, pt] : bs_map) pt.mx_ = DeviceVector<word>();
    std::fill(table.begin(), table.end(), zero_pt_.as<const word>());
    pt_table_.Upload(table);
#endif
  }
}

// Hoist.cu:178-204: the baby and giant steps must be 0, s, 2s, ..., ks
std::pair<int, int> HoistHandler<uint32_t>::CheckStrideMinKS() const {
  AssertTrue(!gs_only_, "Hoist: min_ks should be false for bs == 1 case");
  auto stride = [](auto begin, auto end, const char *what) {
    int count = 0, g = 0, mx = 0;
    for (auto it = begin; it != end; ++it) {
      if (*it == 0) continue;
      g = std::gcd(g, *it);
      count++;
      mx = std::max(mx, *it);
    }
    AssertTrue(count * g == mx, std::string("MinKS does not apply to the "
                                            "given hoist map ") + what);
    return g;
  };
  return {stride(bs_indices_.begin(), bs_indices_.end(), "baby-step sequence"),
          stride(gs_indices_.begin(), gs_indices_.end(),
                 "giant-step sequence")};
}

// Hoist.cu:978-1004
void HoistHandler<uint32_t>::AddRequiredRotations(EvkRequest &req,
                                                  bool min_ks) const {
  for (int r : RequiredRotations(min_ks)) req.AddRequest(r, pt_level_);
}

std::set<int> HoistHandler<uint32_t>::RequiredRotations(bool min_ks) const {
  std::set<int> r;
  if (min_ks) {
    const auto [bs_stride, gs_stride] = CheckStrideMinKS();
    r.insert(bs_stride);
    r.insert(gs_stride);
    return r;
  }
  // a giant-step-only map asks for its giant steps, which here are the
  // baby steps of the converted map: the same set
  for (int b : bs_indices_)
    if (b != 0) r.insert(b);
  for (int g : gs_indices_)
    if (g != 0) r.insert(g);
  return r;
}

void HoistHandler<uint32_t>::Evaluate(ConstContextPtr<word> context, Ct &res,
                                      const Ct &input,
                                      const EvkMap<word> &evk_map,
                                      bool min_ks) const {
  std::map<int, Ct> bs;
  EvaluateBabyStep(context, bs, input, evk_map, min_ks);
  EvaluateGiantStep(context, res, bs, evk_map, min_ks);
}

// src/extension/Hoist.cu:578-691 (hoisted path with BSFusedKeyMult): one
// ModUp of a, then every baby step's key multiply, the PseudoModUp of b and
// the automorphism in one fused launch per CHD_MAX_BS rotations. Results stay
// in the extended basis (q and alpha aux limbs), not divided by P.
void HoistHandler<uint32_t>::EvaluateBabyStep(
    ConstContextPtr<word> context, std::map<int, Ct> &bs, const Ct &input,
    const EvkMap<word> &evk_map, bool min_ks) const {
  BabyStep(
      *context, bs, input,
      [&](int r) { return Context<word>::RefOfKey(evk_map.GetRotationKey(r)); },
      min_ks);
}

void HoistHandler<uint32_t>::EvaluateGiantStep(
    ConstContextPtr<word> context, Ct &res, const std::map<int, Ct> &bs,
    const EvkMap<word> &evk_map, bool min_ks) const {
  GiantStep(
      *context, res, bs,
      [&](int r) { return Context<word>::RefOfKey(evk_map.GetRotationKey(r)); },
      min_ks);
}

namespace {
// HRot at the view level (Context.cpp:776-791): MultKey, then Permute by the
// amount reduced modulo the slot count
void HRotV(const Context<uint32_t> &ctx, int level, uint32_t *res_b,
           uint32_t *res_a, const uint32_t *b, const uint32_t *a,
           const Context<uint32_t>::EvkRef &key, int amount, int slots) {
  const size_t words =
      static_cast<size_t>(ctx.param_.LevelToNP(level).GetNumQ()) *
      ctx.param_.degree_;
  int r = amount % slots;
  if (r < 0) r += slots;
  Workspace::Use use_ws(ctx.GetWorkspace());
  Scratch t(ctx.GetWorkspace(), 2 * words);
  if (r == 0) {
    ctx.PermuteV(level, {res_b, res_a, nullptr}, {b, a, nullptr}, 0);
    return;
  }
  ctx.MultKeyV(level, {t.data(), t.data() + words, nullptr},
               {b, a, nullptr}, key);
  ctx.PermuteV(level, {res_b, res_a, nullptr},
               {t.data(), t.data() + words, nullptr}, r);
}
}  // namespace

// Hoist.cu:517-537: bs[0] = input, bs[k s] = HRot(bs[(k - 1) s], s)
void HoistHandler<uint32_t>::MinKSBabyStep(const Context<word> &ctx,
                                           std::map<int, Ct> &bs,
                                           const Ct &input,
                                           const KeyLookup &key_of) const {
  const int bs_stride = CheckStrideMinKS().first;
  const NPInfo np = input.GetNP();
  const size_t bytes = static_cast<size_t>(np.GetNumQ()) *
                       ctx.param_.degree_ * sizeof(word);
  auto slot = [&](int idx) -> Ct & {
    Ct &ct = bs.try_emplace(idx, np).first->second;
    if (!(ct.GetNP() == np) || ct.HasRx()) ct = Ct(np);
    ct.SetScale(input.GetScale());
    ct.SetNumSlots(input.GetNumSlots());
    return ct;
  };
  for (int b : bs_indices_) {
    Ct &out = slot(b);
    if (b == 0) {
      HipCheck(hipMemcpyAsync(out.bx_.data(), input.bx_.data(), bytes,
                              hipMemcpyDeviceToDevice, CurrentStream()),
               "hipMemcpyAsync");
      HipCheck(hipMemcpyAsync(out.ax_.data(), input.ax_.data(), bytes,
                              hipMemcpyDeviceToDevice, CurrentStream()),
               "hipMemcpyAsync");
      continue;
    }
    auto prev = bs.find(b - bs_stride);
    AssertTrue(prev != bs.end(),
               "Hoist: MinKS baby-step sequence is not complete");
    HRotV(ctx, pt_level_, out.bx_.data(), out.ax_.data(),
          prev->second.bx_.data(), prev->second.ax_.data(), key_of(bs_stride),
          bs_stride, prev->second.GetNumSlots());
  }
}

// Hoist.cu:539-566: giant steps from the last down, each accumulation added
// to the rotated running sum (PAccum with inplace), HRot by the giant-step
// stride unless at giant step 0, then Rescale
void HoistHandler<uint32_t>::MinKSGiantStep(const Context<word> &ctx, Ct &res,
                                            const std::map<int, Ct> &bs,
                                            const KeyLookup &key_of) const {
  const int gs_stride = CheckStrideMinKS().second;
  const Parameter<word> &param = ctx.param_;
  const int n = param.degree_;
  const NPInfo np = param.LevelToNP(pt_level_);
  const size_t qw = static_cast<size_t>(np.GetNumQ()) * n;
  const Ct &ref = bs.begin()->second;
  AssertTrue(ref.GetNP() == np, "Hoist: baby-step level mismatch");
  int num_slots = ref.GetNumSlots();
  for (const auto &[g, pmap] : pt_map_)
    for (const auto &[b, pt] : pmap) {
      AssertTrue(bs.count(b) != 0, "Hoist: missing baby step");
      AssertTrue(bs.at(b).GetNP() == np, "Hoist: baby-step level mismatch");
      num_slots = std::max({num_slots, pt.GetNumSlots(),
                            bs.at(b).GetNumSlots()});
    }
  Workspace *ws = ctx.GetWorkspace();
  Workspace::Use use_ws(ws);
  Scratch acc(ws, 2 * qw);
  // plaintexts held only in the tiled array: each giant step's row is
  // taken back out (its q limbs, one plaintext per baby-step column)
  Scratch row(ws, tiled_rows_ > 0 ? static_cast<size_t>(wide_bs_) * qw : 0);
  const chd_limb_map m = NoSkipMap(param, np);
  bool first = true;
  int prev = 0;
  for (auto it = pt_map_.rbegin(); it != pt_map_.rend(); ++it) {
    const int g = it->first;
    const std::map<int, Pt> &pmap = it->second;
    if (tiled_rows_ > 0) {
      const int gi = static_cast<int>(
          std::find(gs_indices_.begin(), gs_indices_.end(), g) -
          gs_indices_.begin());
      K(chd_k_gs_untile_row(pt_tiled_.as<const word>(), tiled_rows_,
                            wide_bs_, np.GetNumTotal(), gi, np.GetNumQ(),
                            row.data(), CurrentStream()));
    }
    auto pt_of = [&](int b) -> const word * {
      if (tiled_rows_ == 0) return pmap.at(b).mx_.data();
      const auto col = std::distance(bs_indices_.begin(), bs_indices_.find(b));
      return row.data() + static_cast<size_t>(col) * qw;
    };
    // accumulation over this giant step's baby steps (q limbs of each
    // plaintext), onto the rotated running sum after the first
    std::vector<int> bsv;
    for (const auto &[b, pt] : pmap) bsv.push_back(b);
    for (size_t b0 = 0; b0 < bsv.size(); b0 += CHD_GS_MAX_BS) {
      const int bcnt =
          static_cast<int>(std::min<size_t>(CHD_GS_MAX_BS, bsv.size() - b0));
      chd_gs_args a{};
      a.num_bs = bcnt;
      a.num_gs = 1;
      a.add_to_dst = (!first || b0 > 0) ? 1 : 0;
      for (int j = 0; j < bcnt; j++) {
        const Ct &ct = bs.at(bsv[b0 + j]);
        a.bs_b[j] = ct.bx_.data();
        a.bs_a[j] = ct.ax_.data();
        a.pt[0][j] = pt_of(bsv[b0 + j]);
      }
      a.dst_b[0] = acc.data();
      a.dst_a[0] = acc.data() + qw;
      K(chd_k_gs_fused(&ctx.ntt_handler_.Tables(), &m, &a, np.GetNumQ(),
                       CurrentStream()));
    }
    if (!first)
      AssertTrue(prev == g + gs_stride,
                 "Hoist: MinKS giant-step sequence is not complete");
    if (g != 0)
      HRotV(ctx, pt_level_, acc.data(), acc.data() + qw, acc.data(),
            acc.data() + qw, key_of(gs_stride), gs_stride, num_slots);
    else
      AssertTrue(first || prev == gs_stride,
                 "Hoist: MinKS giant-step sequence is not complete");
    first = false;
    prev = g;
  }
  const NPInfo out_np = param.LevelToNP(pt_level_ - 1);
  if (!(res.GetNP() == out_np) ||
      res.bx_.size() != static_cast<size_t>(out_np.GetNumTotal()) * n ||
      res.HasRx())
    res = Ct(out_np);
  ctx.RescaleV(pt_level_, {res.bx_.data(), res.ax_.data(), nullptr},
               {acc.data(), acc.data() + qw, nullptr});
  res.SetNumSlots(num_slots);
  res.SetScale(pt_scale_ * ref.GetScale() /
               param.GetRescalePrimeProd(pt_level_));
}

void HoistHandler<uint32_t>::BabyStep(const Context<word> &ctx,
                                      std::map<int, Ct> &bs, const Ct &input,
                                      const KeyLookup &key_of,
                                      bool min_ks) const {
  const Parameter<word> &param = ctx.param_;
  const int n = param.degree_;
  const NPInfo in_np = input.GetNP();
  AssertTrue(in_np == param.LevelToNP(pt_level_),
             "Hoist: input level mismatch");
  AssertTrue(!input.HasRx(), "Hoist: input should be relinearized");
  // the reference requires an empty bs; here bs may also hold the baby
  // steps of an earlier call, whose buffers are reused when their primes
  // match (no allocation in repeated evaluations)
  for (const auto &[idx, ct] : bs)
    AssertTrue(bs_indices_.count(idx) != 0,
               "Hoist: bs holds a baby step this handler does not use");
  if (min_ks) {
    MinKSBabyStep(ctx, bs, input, key_of);
    return;
  }
  const int num_q = in_np.GetNumQ();
  const int alpha = param.alpha_;
  const int total = num_q + alpha;
  const NPInfo ext_np(in_np.num_main_, in_np.num_ter_, alpha);
  const auto &ms = ctx.mod_switch_handlers_.at(pt_level_);
  // non-empty dnum groups of this level (the first ms.FirstGroup() are
  // skipped with their keys, Context.cpp:637-642)
  const int beta = ms.NumGroups();
  const int first = ms.FirstGroup();
  AssertTrue(beta <= CHD_MAX_BS_GROUPS, "Hoist: dnum too large");
  const DvConstView<word> p_prod = ctx.PProd(in_np);
  Workspace *ws = ctx.GetWorkspace();
  Workspace::Use use_ws(ws);
  std::vector<int> rots;
  for (int b : bs_indices_)
    if (b != 0) rots.push_back(b);
  // 1. ModUp of a, all groups (own limbs are read from a by the kernel)
  const long long gs = static_cast<long long>(total) * n;
  Scratch buf(ws, rots.empty() ? 0
                               : static_cast<size_t>(beta) * gs +
                                     static_cast<size_t>(num_q) * n);
  if (!rots.empty())
    ms.ModUpGroups(buf.data(), gs, input.ax_.ConstView(),
                   buf.data() + beta * gs, true);
  // 2. baby step 0: the PseudoModUp of (b, a), zero on the aux limbs
  auto slot = [&](int idx) -> Ct & {
    Ct &ct = bs.try_emplace(idx, ext_np).first->second;
    if (!(ct.GetNP() == ext_np) ||
        ct.bx_.size() != static_cast<size_t>(total) * n || ct.HasRx())
      ct = Ct(ext_np);
    return ct;
  };
  if (bs_indices_.count(0) != 0) {
    Ct &b0 = slot(0);
    b0.SetScale(input.GetScale());
    b0.SetNumSlots(input.GetNumSlots());
    for (DeviceVector<word> *v : {&b0.bx_, &b0.ax_}) {
      DvView<word> q_part(v->data(), num_q * n, 0);
      const DeviceVector<word> &src = v == &b0.bx_ ? input.bx_ : input.ax_;
      ms.PseudoModUp(q_part, src.ConstView(), p_prod);
      K(chd_k_zero(v->data() + static_cast<size_t>(num_q) * n,
                   static_cast<long long>(alpha) * n, CurrentStream()));
    }
  }
  // 3. the other baby steps, CHD_MAX_BS per fused launch
  const int prime_offset = param.GetMaxNumTer() - in_np.num_ter_;
  chd_limb_map m{};
  m.num_q = num_q;
  m.skip_lo = INT_MAX;
  m.tab_off = param.TerLeft(ext_np);
  m.tab_gap = param.MainLeft(ext_np);
  for (size_t base = 0; base < rots.size(); base += CHD_MAX_BS) {
    chd_bs_args a{};
    a.num_q = num_q;
    a.alpha = alpha;
    a.beta = beta;
    a.group_shift = ms.GroupShift();
    a.modup = buf.data();
    a.group_stride = gs;
    a.d = input.ax_.data();
    a.ct_b = input.bx_.data();
    a.p_prod = p_prod.data();
    const int cnt = static_cast<int>(std::min<size_t>(CHD_MAX_BS, rots.size() - base));
    a.num_rot = cnt;
    for (int k = 0; k < cnt; k++) {
      const int r = rots[base + k];
      const Context<word>::EvkRef key = key_of(r);
      AssertTrue(static_cast<int>(key.bx.size()) >= first + beta &&
                     key.bx.size() == key.ax.size() &&
                     key.np.num_aux_ == alpha,
                 "Hoist: rotation key shape mismatch");
      const long long key_gap =
          static_cast<long long>(key.np.GetNumQ() - prime_offset - num_q) * n;
      AssertTrue(key_gap >= 0, "Hoist: key level below the input level");
      if (k == 0)
        a.key_gap = key_gap;
      else
        AssertTrue(a.key_gap == key_gap, "Hoist: keys of different levels");
      for (int g = 0; g < beta; g++) {
        a.kb[k][g] = key.bx[first + g] + static_cast<size_t>(prime_offset) * n;
        a.ka[k][g] = key.ax[first + g] + static_cast<size_t>(prime_offset) * n;
      }
      // scatter with the inverse automorphism (Hoist.cu:290-300)
      a.galois[k] = static_cast<uint32_t>(param.GetGaloisFactor(n / 2 - r));
      Ct &out = slot(r);
      out.SetScale(input.GetScale());
      out.SetNumSlots(input.GetNumSlots());
      a.dst_b[k] = out.bx_.data();
      a.dst_a[k] = out.ax_.data();
    }
    K(chd_k_bs_fused(&ctx.ntt_handler_.Tables(), &m, &a, CurrentStream()));
  }
}

// src/extension/Hoist.cu:840-975 (EvaluateGiantStepOptimized) and 487-515
// (EvaluateFinalModDown). For every giant step g != 0 the accumulator's a is
// brought down to Q, re-raised and key-multiplied, its b added, and the
// result permuted into the running sum; the b-parts of Hoist.cu's final
// PermuteAccum are folded into the same permuted sum (Permute is linear).
void HoistHandler<uint32_t>::GiantStep(const Context<word> &ctx, Ct &res,
                                       const std::map<int, Ct> &bs,
                                       const KeyLookup &key_of,
                                       bool min_ks) const {
  const Parameter<word> &param = ctx.param_;
  const int n = param.degree_;
  AssertTrue(!bs.empty(), "Hoist: bs should not be empty");
  if (min_ks) {
    MinKSGiantStep(ctx, res, bs, key_of);
    return;
  }
  const Ct &ref = bs.begin()->second;
  const NPInfo ext_np = ref.GetNP();
  const int alpha = param.alpha_;
  AssertTrue(ext_np.num_aux_ == alpha, "Hoist: baby steps must be extended");
  AssertTrue(param.NPToLevel(NPInfo(ext_np.num_main_, ext_np.num_ter_, 0)) ==
                 pt_level_,
             "Hoist: baby-step level mismatch");
  const int num_q = ext_np.GetNumQ();
  const int total = num_q + alpha;
  const size_t tw = static_cast<size_t>(total) * n;
  const double input_scale = ref.GetScale();
  int num_slots = ref.GetNumSlots();
  for (const auto &[g, pmap] : pt_map_)
    for (const auto &[b, pt] : pmap) {
      AssertTrue(bs.count(b) != 0, "Hoist: missing baby step");
      num_slots = std::max({num_slots, pt.GetNumSlots(),
                            bs.at(b).GetNumSlots()});
    }
  const auto &ms = ctx.mod_switch_handlers_.at(pt_level_);
  Workspace *ws = ctx.GetWorkspace();
  Workspace::Use use_ws(ws);
  chd_limb_map m = NoSkipMap(param, ext_np);
  // 1. every giant step's plaintext accumulation (GSFusedPAccum,
  //    Hoist.cu:334-445): one fused launch per CHD_GS_MAX_GS giant steps and
  //    CHD_GS_MAX_BS baby steps, each baby step read once per launch
  const int num_gs = static_cast<int>(gs_indices_.size());
  const std::vector<int> bsv(bs_indices_.begin(), bs_indices_.end());
  Scratch accs(ws, static_cast<size_t>(num_gs) * 2 * tw);
  auto acc_b = [&](int gi) { return accs.data() + static_cast<size_t>(gi) * 2 * tw; };
  if (wide_gs_ > 0) {
    // every giant step in one launch: each baby step is read once
    // (plaintext addresses from the handler's table; baby steps padded to
    // wide_bs_ with the zero plaintext)
    chd_gs_wide_args a{};
    a.num_bs = wide_bs_;
    a.num_gs = wide_gs_;
    a.add_to_dst = 0;
    a.pt_stride = wide_bs_;
    a.pt_table = pt_table_.as<const word *>();
    a.pt_tiled = tiled_rows_ > 0 ? pt_tiled_.as<const word>() : nullptr;
    a.tiled_rows = tiled_rows_;
    for (int j = 0; j < wide_bs_; j++) {
      const bool real = j < static_cast<int>(bsv.size());
      a.bs_b[j] = real ? bs.at(bsv[j]).bx_.data() : zero_pt_.as<word>();
      a.bs_a[j] = real ? bs.at(bsv[j]).ax_.data() : zero_pt_.as<word>();
    }
    for (int k = 0; k < wide_gs_; k++) {
      a.dst_b[k] = k < num_gs ? acc_b(k) : dummy_out_.as<word>();
      a.dst_a[k] = k < num_gs ? acc_b(k) + tw : dummy_out_.as<word>() + tw;
    }
    K(chd_k_gs_fused_wide(&ctx.ntt_handler_.Tables(), &m, &a, total,
                          CurrentStream()));
  }
  for (int g0 = 0; wide_gs_ == 0 && g0 < num_gs; g0 += CHD_GS_MAX_GS) {
    const int gcnt = std::min(CHD_GS_MAX_GS, num_gs - g0);
    for (size_t b0 = 0; b0 < bsv.size(); b0 += CHD_GS_MAX_BS) {
      const int bcnt = static_cast<int>(
          std::min<size_t>(CHD_GS_MAX_BS, bsv.size() - b0));
      chd_gs_args a{};
      a.num_bs = bcnt;
      a.num_gs = gcnt;
      a.add_to_dst = b0 > 0 ? 1 : 0;
      for (int j = 0; j < bcnt; j++) {
        const Ct &ct = bs.at(bsv[b0 + j]);
        a.bs_b[j] = ct.bx_.data();
        a.bs_a[j] = ct.ax_.data();
      }
      for (int k = 0; k < gcnt; k++) {
        const std::map<int, Pt> &pmap = pt_map_.at(gs_indices_[g0 + k]);
        for (int j = 0; j < bcnt; j++) {
          auto it = pmap.find(bsv[b0 + j]);
          a.pt[k][j] = it == pmap.end() ? nullptr : it->second.mx_.data();
        }
        a.dst_b[k] = acc_b(g0 + k);
        a.dst_a[k] = acc_b(g0 + k) + tw;
      }
      K(chd_k_gs_fused(&ctx.ntt_handler_.Tables(), &m, &a, total,
                       CurrentStream()));
    }
  }
  // 2. giant-step rotations (EvaluateGiantStepOptimized, Hoist.cu:895-957):
  //    fin = acc_0 + sum_{g != 0} Permute(KS(ModUp(ModDown(acc_g.a))) with
  //    acc_g.b added, g)
  // giant step 0 (the first, indices ascend) accumulates in place. The
  // other giant steps are independent until their permuted sum, so they
  // run in batches of up to CHD_MAX_JOBS: one ModDown, one ModUp, one key
  // accumulation and one permute-accumulate launch sequence per batch
  // (modular sums, so the batching leaves every residue as it was).
  const bool has0 = gs_indices_.front() == 0;
  const int first_gi = has0 ? 1 : 0;
  const int batch = std::max(1, std::min(CHD_MAX_JOBS, num_gs - first_gi));
  Scratch fin_buf(ws, has0 ? 0 : 2 * tw),
      tmp(ws, static_cast<size_t>(batch) * 2 * tw),
      down(ws, static_cast<size_t>(batch) * num_q * n);
  word *const finp = has0 ? acc_b(0) : fin_buf.data();
  bool first = !has0;
  const long long dlen = static_cast<long long>(num_q) * n;
  for (int g0 = first_gi; g0 < num_gs; g0 += batch) {
    const int cnt = std::min(batch, num_gs - g0);
    // ModDown of every accumulator's a (acc_a of giant step gi sits at
    // acc_b(gi) + tw, 2 tw words apart)
    std::vector<word *> dd(cnt);
    for (int i = 0; i < cnt; i++) dd[i] = down.data() + i * dlen;
    ms.ModDownMulti(dd, acc_b(g0) + tw, static_cast<long long>(2 * tw),
                    ModSwitchHandler<word>::Kind::ModDown);
    std::vector<Context<word>::EvkRef> keys;
    keys.reserve(cnt);
    const Context<word>::EvkRef *kp[CHD_MAX_JOBS];
    word *tb[CHD_MAX_JOBS], *ta[CHD_MAX_JOBS];
    chd_perm_src ps[CHD_MAX_JOBS] = {};
    for (int i = 0; i < cnt; i++) {
      const int g = gs_indices_[g0 + i];
      keys.push_back(key_of(g));
      tb[i] = tmp.data() + static_cast<size_t>(i) * 2 * tw;
      ta[i] = tb[i] + tw;
      ps[i].src[0] = tb[i];
      ps[i].src[1] = ta[i];
      ps[i].galois = ctx.elem_handler_.PermuteAmountToGaloisFactor(g);
    }
    for (int i = 0; i < cnt; i++) kp[i] = &keys[i];
    ctx.KeyMultExtBatchV(pt_level_, cnt, tb, ta, down.data(), dlen,
                         acc_b(g0), static_cast<long long>(2 * tw), kp);
    word *dp[2] = {finp, finp + tw};
    const word *s0[2] = {finp, finp + tw};
    K(chd_k_permute_accum(&ctx.ntt_handler_.Tables(), &m, dp, 2,
                          first ? nullptr : s0, 0, ps, cnt, total,
                          CurrentStream()));
    first = false;
  }
  // EvaluateFinalModDown: merged ModDown and rescale of both polynomials,
  // into res's own buffers when they already have the output's primes
  const NPInfo out_np = param.LevelToNP(pt_level_ - 1);
  if (!(res.GetNP() == out_np) ||
      res.bx_.size() != static_cast<size_t>(out_np.GetNumTotal()) * n ||
      res.HasRx())
    res = Ct(out_np);
  ms.ModDownMulti({res.bx_.data(), res.ax_.data()}, finp,
                  static_cast<long long>(tw),
                  ModSwitchHandler<word>::Kind::ModDownAndRescale);
  res.SetNumSlots(num_slots);
  res.SetScale(pt_scale_ * input_scale / param.GetRescalePrimeProd(pt_level_));
}

// ------------------------------------------------------- StripedMatrix --
// src/extension/StripedMatrix.cpp:17-47
StripedMatrix StripedMatrix::Mult(const StripedMatrix &a,
                                  const StripedMatrix &b) {
  AssertTrue(a.width_ == a.height_ && b.width_ == b.height_,
             "StripedMatrix must be square to perform multiplication");
  AssertTrue(a.GetHeight() == b.GetWidth(), "StripedMatrix dimension mismatch");
  const int w = a.width_;
  StripedMatrix c(w, w);
  for (const auto &[i, da] : a)
    for (const auto &[j, db] : b) {
      std::vector<Complex> &dc =
          c.try_emplace((i + j) % w, std::vector<Complex>(w)).first->second;
      for (int k = 0; k < w; k++) dc[k] += da[k] * db[(k + i) % w];
    }
  return c;
}

StripedMatrix StripedMatrix::Mult(const StripedMatrix &a, const Complex b) {
  StripedMatrix c(a.GetHeight(), a.GetWidth());
  for (const auto &[i, d] : a) {
    std::vector<Complex> &dc = c.try_emplace(i, d.size()).first->second;
    for (size_t j = 0; j < d.size(); j++) dc[j] = d[j] * b;
  }
  return c;
}

// ----------------------------------------------------- LinearTransform --
// src/extension/LinearTransform.cpp:9-38: the gcd of the diagonals' rotation
// amounts after the pre-rotation
int LinearTransform<uint32_t>::DetermineStride(const StripedMatrix &matrix,
                                               int bs, int gs,
                                               int pre_rotation) {
  const int width = matrix.GetWidth();
  AssertTrue(width > 0, "LinearTransform requires a positive width");
  int gcd_rot = 0, max_rot = 0, num_pt = 0;
  for (const auto &[i, diag] : matrix) {
    num_pt++;
    int rot = (i - pre_rotation) % width;
    if (rot < 0) rot += width;
    gcd_rot = std::gcd(gcd_rot, rot);
    max_rot = std::max(max_rot, rot);
  }
  AssertTrue(num_pt > 1, "LinearTransform requires at least 2 plaintexts");
  AssertTrue(gcd_rot > 0, "Something went wrong during LinearTransform setup");
  AssertTrue(max_rot <= (bs * gs - 1) * gcd_rot,
             "Incompatible matrix and LinearTransform parameters: bs (" +
                 std::to_string(bs) + "), gs (" + std::to_string(gs) +
                 "), pre_rotation (" + std::to_string(pre_rotation) + ")");
  return gcd_rot;
}

// LinearTransform.cpp:40-72: diagonal rot = gs_rot + bs_rot with bs_rot below
// stride * bs; its message is the diagonal rotated right by
// gs_rot - additional_pt_rot (the giant step's rotation undone ahead)
HoistHandler<uint32_t>::PlainHoistMap
LinearTransform<uint32_t>::ConstructPlainHoistMap(const StripedMatrix &matrix,
                                                  int bs, int gs,
                                                  int pre_rotation,
                                                  int additional_pt_rot) {
  const int height = matrix.GetHeight();
  const int width = matrix.GetWidth();
  auto pow2 = [](int v) {
    AssertTrue(v > 0, "IsPowOfTwo only accepts positive values");
    return (v & (v - 1)) == 0;
  };
  AssertTrue(pow2(height), "LinearTransform requires power-of-two height");
  AssertTrue(pow2(width), "LinearTransform requires power-of-two width");
  AssertTrue(height == width, "LinearTransform requires square matrix");
  const int gs_stride = DetermineStride(matrix, bs, gs, pre_rotation) * bs;
  HoistHandler<word>::PlainHoistMap map;
  for (const auto &[i, diag] : matrix) {
    AssertTrue(static_cast<int>(diag.size()) >= height,
               "LinearTransform: diagonal shorter than the matrix");
    int rot = (i - pre_rotation) % width;
    if (rot < 0) rot += width;
    const int bs_rot = rot % gs_stride;
    const int gs_rot = rot - bs_rot;
    std::vector<Complex> &msg =
        map[gs_rot].try_emplace(bs_rot, height, Complex(0)).first->second;
    int offset = (gs_rot - additional_pt_rot) % height;
    if (offset < 0) offset += height;
    for (int j = 0; j < height; j++) msg[(j + offset) % height] = diag[j];
  }
  return map;
}

// LinearTransform.cpp:74-88
LinearTransform<uint32_t>::LinearTransform(ConstContextPtr<word> context,
                                           const StripedMatrix &matrix,
                                           int pt_level, double pt_scale,
                                           int bs, int gs, int pre_rotation,
                                           int additional_pt_rot)
    : bs_(bs),
      gs_(gs),
      pre_rotation_(pre_rotation),
      hoist_(context,
             ConstructPlainHoistMap(matrix, bs, gs, pre_rotation,
                                    additional_pt_rot),
             pt_level, pt_scale) {}

}  // namespace cheddar
