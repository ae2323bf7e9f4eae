// C++ host API of the MI355X key-switch path, mirroring the reference's
// classes and entry points so existing callers compile against it:
//   Parameter          include/core/Parameter.h:22-253
//   NPInfo             include/core/NPInfo.h
//   DvView/DeviceVector include/core/DeviceVector.h:27-125
//   Ciphertext/EvaluationKey include/core/Container.h:132-345
//   NTTHandler         include/core/NTT.h:56-81
//   ModSwitchHandler   include/core/ModSwitch.h:40-44
//   ElementWiseHandler include/core/ElementWise.h:88-109 (key-switch subset)
//   Context            include/core/Context.h:70-423 (key-switch subset)
// Only word = uint32_t is provided, N = 2^16, no terminal primes (a
// Parameter with terminal primes is rejected with an error).
// Failures throw cheddar::Error (the reference prints and exits); the C-ABI
// (include/cheddar_amd.h) converts them into status codes.
// Kernels are reached through the kernel C-ABI (include/cheddar_kernels.h).
#pragma once

#include <hip/hip_runtime.h>

#include <complex>
#include <cstdint>
#include <memory>
#include <functional>
#include <map>
#include <mutex>
#include <set>
#include <unordered_map>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "cheddar_kernels.h"
#include "device_tables.h"
#include "memory_pool.h"

namespace cheddar {

struct Error : std::runtime_error {
  explicit Error(const std::string &m) : std::runtime_error(m) {}
};
inline void AssertTrue(bool c, const std::string &msg) {
  if (!c) throw Error("ERROR: " + msg);
}
// literal messages: no string is built unless the check fails
inline void AssertTrue(bool c, const char *msg) {
  if (!c) throw Error(std::string("ERROR: ") + msg);
}
[[noreturn]] inline void Fail(const std::string &msg) {
  throw Error("ERROR: " + msg);
}

// Stream the library launches on (the reference uses the legacy default
// stream; the C-ABI sets the caller's stream for the duration of a call).
hipStream_t CurrentStream();
class StreamScope {
 public:
  explicit StreamScope(hipStream_t s);
  ~StreamScope();

 private:
  hipStream_t prev_;
};

struct NPInfo {
  int num_main_ = 0;
  int num_ter_ = 0;
  int num_aux_ = 0;
  explicit NPInfo(int num_main = 0, int num_ter = 0, int num_aux = 0);
  int GetNumQ() const { return num_main_ + num_ter_; }
  int GetNumTotal() const { return num_main_ + num_ter_ + num_aux_; }
  bool operator==(const NPInfo &o) const {
    return num_main_ == o.num_main_ && num_ter_ == o.num_ter_ &&
           num_aux_ == o.num_aux_;
  }
  bool IsSubsetOf(const NPInfo &o) const {
    return num_main_ <= o.num_main_ && num_ter_ <= o.num_ter_ &&
           num_aux_ <= o.num_aux_;
  }
};

template <typename word>
class Parameter;

template <>
class Parameter<uint32_t> {
 public:
  using word = uint32_t;
  Parameter(int log_degree, double base_scale, int default_encryption_level,
            std::vector<std::pair<int, int>> level_config,
            const std::vector<word> &main_primes,
            const std::vector<word> &aux_primes,
            const std::vector<word> &ter_primes = std::vector<word>{},
            const std::pair<int, int> &additional_base = {0, 0});

  const int log_degree_;
  const int degree_;
  const int dnum_;
  const int L_;
  const int alpha_;
  const double base_scale_;
  const int default_encryption_level_;
  const int max_level_;

  NPInfo LevelToNP(int level, int num_aux = 0) const;
  int NPToLevel(const NPInfo &np) const;
  std::vector<word> GetPrimeVector(const NPInfo &np) const;
  int GetMaxNumMain() const { return static_cast<int>(main_primes_.size()); }
  int GetMaxNumTer() const { return static_cast<int>(ter_primes_.size()); }
  int GetMaxNumAux() const { return alpha_; }
  int GetGaloisFactor(int rot) const;
  double GetScale(int level) const;
  double GetRescalePrimeProd(int level) const;
  // chain position of limb 0 of np / aux gap (the reference's ter_left and
  // main_left, src/core/NTT.cu:620-621)
  int TerLeft(const NPInfo &np) const { return GetMaxNumTer() - np.num_ter_; }
  int MainLeft(const NPInfo &np) const {
    return GetMaxNumMain() - np.num_main_;
  }
  // the full chain: ter reversed, main, aux (Parameter.cu:103-111)
  const std::vector<word> &ChainPrimes() const { return chain_; }

 private:
  std::vector<word> main_primes_, ter_primes_, aux_primes_;
  std::vector<std::pair<int, int>> level_config_;
  std::vector<word> chain_;
  std::vector<int> galois_factors_;
  std::vector<double> scale_, rescale_prime_prod_;
};

// A parameter set from the reference's JSON layout (parameters/*.json as
// unittest/Testbed.h:95-179 reads it); throws Error on a malformed file or
// an unsupported set.
std::unique_ptr<Parameter<uint32_t>> ParameterFromJson(
    const std::string &text);

// Non-owning views: (pointer, total words, aux words) (DeviceVector.h:27-72)
template <typename word>
class DvView {
 public:
  DvView(word *p = nullptr, int total = 0, int aux = 0)
      : p_(p), total_(total), aux_(aux) {}
  word *data() const { return p_; }
  int TotalSize() const { return total_; }
  int AuxSize() const { return aux_; }
  int QSize() const { return total_ - aux_; }

 private:
  word *p_;
  int total_, aux_;
};

template <typename word>
class DvConstView {
 public:
  DvConstView(const word *p = nullptr, int total = 0, int aux = 0)
      : p_(p), total_(total), aux_(aux) {}
  DvConstView(const DvView<word> &v)  // NOLINT: implicit like the reference
      : p_(v.data()), total_(v.TotalSize()), aux_(v.AuxSize()) {}
  const word *data() const { return p_; }
  int TotalSize() const { return total_; }
  int AuxSize() const { return aux_; }
  int QSize() const { return total_ - aux_; }

 private:
  const word *p_;
  int total_, aux_;
};

// Owning device vector (include/core/DeviceVector.h:80-125): memory from
// the device's MemoryPool, taken and given back in the order of the stream
// current when it is (re)allocated, as the reference's rmm::device_uvector
// takes it from its pool on its stream. resize keeps the first
// min(old, new) words and reallocates only beyond the capacity.
template <typename word>
class DeviceVector {
 public:
  DeviceVector() = default;
  explicit DeviceVector(size_t n) { resize(n); }
  ~DeviceVector() { Free(); }
  DeviceVector(const DeviceVector &) = delete;
  DeviceVector &operator=(const DeviceVector &) = delete;
  DeviceVector(DeviceVector &&o) noexcept
      : p_(o.p_),
        n_(o.n_),
        reserved_(o.reserved_),
        stream_(o.stream_),
        pool_(o.pool_) {
    o.p_ = nullptr;
    o.n_ = o.reserved_ = 0;
  }
  DeviceVector &operator=(DeviceVector &&o) noexcept {
    if (this != &o) {
      Free();
      p_ = o.p_;
      n_ = o.n_;
      reserved_ = o.reserved_;
      stream_ = o.stream_;
      pool_ = o.pool_;
      o.p_ = nullptr;
      o.n_ = o.reserved_ = 0;
    }
    return *this;
  }
  void resize(size_t n) {
    if (n * sizeof(word) <= reserved_) {
      n_ = n;
      return;
    }
    const hipStream_t s = CurrentStream();
    size_t reserved = 0;
    MemoryPool &pool = MemoryPool::Current();
    word *p = static_cast<word *>(pool.Allocate(n * sizeof(word), s,
                                                &reserved));
    if (n_ != 0) {
      const hipError_t e = hipMemcpyAsync(p, p_, n_ * sizeof(word),
                                          hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) {
        pool.Deallocate(p, reserved, s);
        HipCheck(e, "hipMemcpyAsync");
      }
    }
    // the old block's last use is the copy above, on s
    if (p_ != nullptr) pool_->Deallocate(p_, reserved_, s);
    p_ = p;
    n_ = n;
    reserved_ = reserved;
    stream_ = s;
    pool_ = &pool;
  }
  // gives the memory back (the reference's shrink_to_fit of an empty vector)
  void shrink_to_fit() {
    if (n_ == 0) Free();
  }
  // DeviceVector.cpp:75-85: size more words, the new ones zero
  void ZeroExtend(size_t size) {
    if (size == 0) return;
    const size_t old = n_;
    resize(old + size);
    HipCheck(hipMemsetAsync(p_ + old, 0, size * sizeof(word), stream_),
             "hipMemsetAsync");
  }
  hipStream_t stream() const { return stream_; }
  size_t size() const { return n_; }
  size_t capacity() const { return reserved_ / sizeof(word); }
  word *data() { return p_; }
  const word *data() const { return p_; }
  DvView<word> View(int aux_size = 0, int front = 0) {
    return DvView<word>(data() + front, static_cast<int>(n_) - front, aux_size);
  }
  DvConstView<word> ConstView(int aux_size = 0, int front = 0) const {
    return DvConstView<word>(data() + front, static_cast<int>(n_) - front,
                             aux_size);
  }

 private:
  void Free() noexcept {
    if (p_ != nullptr) pool_->Deallocate(p_, reserved_, stream_);
    p_ = nullptr;
    n_ = reserved_ = 0;
  }
  word *p_ = nullptr;
  size_t n_ = 0, reserved_ = 0;
  hipStream_t stream_ = nullptr;
  MemoryPool *pool_ = nullptr;  // the pool of the device it came from
};

// the reference's host-side vector (DeviceVector.h:15, a thrust host_vector)
template <typename word>
using HostVector = std::vector<word>;

// DeviceVector.cpp:101-125: copies in the destination's stream order (the
// host side must stay valid until the copy has run)
template <typename word>
void CopyHostToDevice(DeviceVector<word> &dst, const std::vector<word> &src) {
  dst.resize(src.size());
  HipCheck(hipMemcpyAsync(dst.data(), src.data(), src.size() * sizeof(word),
                          hipMemcpyHostToDevice, dst.stream()),
           "hipMemcpyAsync");
}
template <typename word>
void CopyDeviceToHost(std::vector<word> &dst, const DeviceVector<word> &src) {
  dst.resize(src.size());
  HipCheck(hipMemcpyAsync(dst.data(), src.data(), src.size() * sizeof(word),
                          hipMemcpyDeviceToHost, src.stream()),
           "hipMemcpyAsync");
}
template <typename word>
void CopyDeviceToDevice(DeviceVector<word> &dst,
                        const DeviceVector<word> &src) {
  dst.resize(src.size());
  if (src.data() == dst.data()) return;
  HipCheck(hipMemcpyAsync(dst.data(), src.data(), src.size() * sizeof(word),
                          hipMemcpyDeviceToDevice, dst.stream()),
           "hipMemcpyAsync");
}

// Device scratch arena of one Context. Key-switch temporaries (the
// reference's per-call RMM allocations, ModSwitch.cu:442,597;
// Context.cpp:670-682) are carved from it in LIFO order with a bump pointer:
// stream-ordered allocation costs tens of microseconds of host time per call
// on this runtime, more than some of the kernels it feeds. The arena serves
// one stream at a time: a call on a different stream than the previous call
// first makes its stream wait for the event recorded at the end of that call.
// Calls from several host threads are serialised by a mutex.
class Workspace {
 public:
  explicit Workspace(size_t words);
  ~Workspace();
  Workspace(const Workspace &) = delete;
  Workspace &operator=(const Workspace &) = delete;
  // Guard for one API call that takes scratch from the arena (re-entrant).
  class Use {
   public:
    explicit Use(Workspace *ws);
    ~Use();
    Use(const Use &) = delete;
    Use &operator=(const Use &) = delete;

   private:
    Workspace *ws_;
  };
  // For one guarded call, temporaries come from caller-given device memory
  // [base, base + words) instead of the arena, and running out of it throws
  // instead of allocating. Taken inside a Use guard of this workspace with
  // no temporary live; the arena is back when the guard ends.
  class External {
   public:
    External(Workspace *ws, uint32_t *base, size_t words);
    ~External();
    External(const External &) = delete;
    External &operator=(const External &) = delete;

   private:
    Workspace *ws_;
    uint32_t *saved_base_;
    size_t saved_cap_;
  };
  // nullptr when the arena has no room left
  uint32_t *Push(size_t words);
  void Pop(uint32_t *p);
  size_t Capacity() const { return cap_; }
  // no fallback allocation allowed (an External guard is active)
  bool Strict() const { return strict_; }

 private:
  void Enter();
  void Leave() noexcept;
  DevBuf buf_;
  uint32_t *base_ = nullptr;
  bool strict_ = false;
  size_t cap_ = 0, top_ = 0;
  int depth_ = 0;
  hipEvent_t done_ = nullptr;
  hipStream_t cur_ = nullptr, last_ = nullptr;
  bool has_last_ = false;
  std::recursive_mutex mu_;
};

// A temporary of `words` words: from the arena when one is given and has
// room, otherwise stream-ordered (hipMallocAsync / hipFreeAsync on the
// current stream), or an Error when the workspace is strict. Must be
// released in LIFO order (automatic scope).
class Scratch {
 public:
  Scratch(Workspace *ws, size_t words);
  explicit Scratch(size_t words) : Scratch(nullptr, words) {}
  ~Scratch();
  Scratch(const Scratch &) = delete;
  Scratch &operator=(const Scratch &) = delete;
  uint32_t *data() const { return p_; }

 private:
  uint32_t *p_ = nullptr;
  Workspace *ws_ = nullptr;
  hipStream_t s_ = nullptr;
};

template <typename word>
class Ciphertext;
template <>
class Ciphertext<uint32_t> {
 public:
  using word = uint32_t;
  explicit Ciphertext(const NPInfo &np = NPInfo{}, bool has_rx = false);
  DeviceVector<word> bx_, ax_, rx_;
  bool HasRx() const { return rx_.size() != 0; }
  void PrepareRx();
  void RemoveRx();
  NPInfo GetNP() const { return np_; }
  void ModifyNP(const NPInfo &np);
  int GetNumSlots() const { return num_slots_; }
  void SetNumSlots(int n) { num_slots_ = n; }
  double GetScale() const { return scale_; }
  void SetScale(double s) { scale_ = s; }
  static void SetDegree(int degree) { degree_ = degree; }

 private:
  static inline int degree_ = 1 << 16;
  NPInfo np_;
  int num_slots_ = (1 << 16) / 2;
  double scale_ = 1.0;
};

template <typename word>
class EvaluationKey;
template <>
class EvaluationKey<uint32_t> {
 public:
  using word = uint32_t;
  EvaluationKey(const NPInfo &np, int beta, int degree = 1 << 16);
  std::vector<DeviceVector<word>> bx_, ax_;
  int GetBeta() const { return static_cast<int>(bx_.size()); }
  NPInfo GetNP() const { return np_; }

 private:
  NPInfo np_;
};

// Plaintext (include/core/Container.h:226-270): one polynomial mx_ in the
// NTT domain (Montgomery form), with its primes, scale and slot count.
template <typename word>
class Plaintext;
template <>
class Plaintext<uint32_t> {
 public:
  using word = uint32_t;
  explicit Plaintext(const NPInfo &np = NPInfo{}, int degree = 1 << 16);
  DeviceVector<word> mx_;
  NPInfo GetNP() const { return np_; }
  int GetNumSlots() const { return num_slots_; }
  void SetNumSlots(int n) { num_slots_ = n; }
  double GetScale() const { return scale_; }
  void SetScale(double s) { scale_ = s; }

 private:
  NPInfo np_;
  int num_slots_ = (1 << 16) / 2;
  double scale_ = 1.0;
};

// Constant (include/core/Container.h:72-130): one residue per prime, in
// Montgomery form, with its scale.
template <typename word>
class Constant;
template <>
class Constant<uint32_t> {
 public:
  using word = uint32_t;
  explicit Constant(const NPInfo &np = NPInfo{});
  DeviceVector<word> cx_;
  NPInfo GetNP() const { return np_; }
  double GetScale() const { return scale_; }
  void SetScale(double s) { scale_ = s; }

 private:
  NPInfo np_;
  double scale_ = 1.0;
};

// Rotation-key container (include/core/EvkMap.h): evaluation keys by index.
template <typename word>
class EvkMap;
template <>
class EvkMap<uint32_t>
    : public std::unordered_map<int, EvaluationKey<uint32_t>> {
 public:
  using Base = std::unordered_map<int, EvaluationKey<uint32_t>>;
  using Base::Base;
  EvkMap() = default;
  EvkMap(const EvkMap &) = delete;
  EvkMap &operator=(const EvkMap &) = delete;
  EvkMap(EvkMap &&) = default;
  const EvaluationKey<uint32_t> &GetRotationKey(int rot_idx) const;
};

// Rotation-key request (include/core/EvkRequest.h, src/core/EvkRequest.cpp):
// rotation index -> the highest level a key is needed at.
class EvkRequest : public std::map<int, int> {
 public:
  using Base = std::map<int, int>;
  using Base::Base;
  void AddRequest(int rot_idx, int level);
};

template <typename word>
class NTTHandler;
template <>
class NTTHandler<uint32_t> {
 public:
  using word = uint32_t;
  explicit NTTHandler(const Parameter<word> &param);
  void NTT(DvView<word> &dst, const NPInfo &np, const DvConstView<word> &src,
           bool montgomery_conversion = false) const;
  void INTT(DvView<word> &dst, const NPInfo &np, const DvConstView<word> &src,
            bool montgomery_conversion = true) const;
  void INTTAndMultConst(DvView<word> &dst, const NPInfo &np,
                        const DvConstView<word> &src,
                        const DvConstView<word> &src_const,
                        bool normalize = false) const;
  void NTTForModUp(DvView<word> &dst, const NPInfo &np, int skip_start,
                   int skip_end, const DvConstView<word> &src) const;
  void NTTForModDown(DvView<word> &dst, const NPInfo &np_src1,
                     const NPInfo &np_src2, const DvConstView<word> &src1,
                     const DvConstView<word> &src2,
                     const DvConstView<word> &inv_p_prod,
                     const DvConstView<word> &src2_padding =
                         DvConstView<word>(nullptr, 0)) const;
  void INTTForModDown(DvView<word> &dst, const NPInfo &np_src,
                      const NPInfo &np_non_intt, const DvConstView<word> &src,
                      const DvConstView<word> &src_const) const;
  const chd_tables &Tables() const { return chain_.tables(); }

 private:
  chd_limb_map Map(const NPInfo &np) const;
  const Parameter<word> &param_;
  ChainTables chain_;
};

template <typename word>
class ElementWiseHandler;
template <>
class ElementWiseHandler<uint32_t> {
 public:
  using word = uint32_t;
  ElementWiseHandler(const Parameter<word> &param,
                     const NTTHandler<word> &ntt);
  void Tensor(std::vector<DvView<word>> &dst, const NPInfo &np,
              const std::vector<DvConstView<word>> &src1,
              const std::vector<DvConstView<word>> &src2) const;
  void PAccum(std::vector<DvView<word>> &dst, const NPInfo &np,
              const std::vector<std::vector<DvConstView<word>>> &ct_srcs,
              const std::vector<DvConstView<word>> &common_srcs) const;
  void CAccum(std::vector<DvView<word>> &dst, const NPInfo &np,
              const std::vector<std::vector<DvConstView<word>>> &ct_srcs,
              const std::vector<DvConstView<word>> &common_srcs) const;
  void Permute(std::vector<DvView<word>> &dst, const NPInfo &np,
               int permute_amount,
               const std::vector<DvConstView<word>> &src1) const;
  uint32_t PermuteAmountToGaloisFactor(int permute_amount) const;
  // ElementWise.cu:1002-1110: dst = sum_i Permute(srcs[i], amounts[i]), plus
  // srcs.back() unpermuted when srcs has one entry more than amounts
  void PermuteAccum(std::vector<DvView<word>> &dst, const NPInfo &np,
                    const std::vector<int> &permute_amounts,
                    const std::vector<std::vector<DvConstView<word>>> &srcs)
      const;
  // ElementWise.cu:687-920, 1673-1706 (canonical residues in and out)
  using Views = std::vector<DvView<word>>;
  using CViews = std::vector<DvConstView<word>>;
  void Add(Views &dst, const NPInfo &np, const CViews &src1,
           const CViews &src2) const;
  void Sub(Views &dst, const NPInfo &np, const CViews &src1,
           const CViews &src2) const;
  void Neg(Views &dst, const NPInfo &np, const CViews &src1) const;
  void Mult(Views &dst, const NPInfo &np, const CViews &src1,
            const CViews &src2) const;
  void PMult(Views &dst, const NPInfo &np, const CViews &src1,
             const DvConstView<word> &src2) const;
  void AddConst(Views &dst, const NPInfo &np, const CViews &src1,
                const DvConstView<word> &src_const) const;
  void SubConst(Views &dst, const NPInfo &np, const CViews &src1,
                const DvConstView<word> &src_const) const;
  // dst = const - src1
  void SubOppositeConst(Views &dst, const NPInfo &np, const CViews &src1,
                        const DvConstView<word> &src_const) const;
  void MultConst(Views &dst, const NPInfo &np, const CViews &src1,
                 const DvConstView<word> &src_const) const;
  // multiplication by X^(N/2), the imaginary unit of the slots
  void MultImaginaryUnit(Views &dst, const NPInfo &np,
                         const CViews &src1) const;
  void Copy(Views &dst, const NPInfo &np, const CViews &src1) const;

 private:
  void Elementwise(int op, Views &dst, const NPInfo &np, const CViews &src1,
                   const CViews *src2, const DvConstView<word> *cst) const;
  void CPAccumWorker(bool const_accum, std::vector<DvView<word>> &dst,
                     const NPInfo &np,
                     const std::vector<std::vector<DvConstView<word>>> &ct_srcs,
                     const std::vector<DvConstView<word>> &common_srcs) const;
  const Parameter<word> &param_;
  const NTTHandler<word> &ntt_;
};

template <typename word>
class ModSwitchHandler;
template <>
class ModSwitchHandler<uint32_t> {
 public:
  using word = uint32_t;
  ModSwitchHandler(const Parameter<word> &param, int level,
                   const ElementWiseHandler<word> &elem,
                   const NTTHandler<word> &ntt, Workspace *ws = nullptr);
  void ModUp(std::vector<DvView<word>> &dst,
             const DvConstView<word> &src) const;
  void ModDown(DvView<word> &dst, const DvConstView<word> &src) const;
  void Rescale(DvView<word> &dst, const DvConstView<word> &src) const;
  void ModDownAndRescale(DvView<word> &dst,
                         const DvConstView<word> &src) const;
  int GetBeta() const { return beta_; }
  // dnum groups sit on the chain's positions (ModSwitch.cu:200-235): with
  // terminal primes missing at this level, the first FirstGroup() groups are
  // empty; non-empty group z (0 <= z < NumGroups(), chain group
  // FirstGroup() + z) owns the level's limbs [GroupLo(z), GroupHi(z)).
  int FirstGroup() const { return first_group_; }
  int NumGroups() const { return beta_ - first_group_; }
  int GroupShift() const { return group_shift_; }
  int GroupLo(int z) const;
  int GroupHi(int z) const;
  // ModSwitch.cu:414-428: dst = MontMul(src, p_prod) on the q limbs
  void PseudoModUp(DvView<word> &dst, const DvConstView<word> &src,
                   const DvConstView<word> &p_prod) const;

  // Batched pieces of ModUp used by the fused key switch (no single
  // reference counterpart). ModUpBconv: INTTAndMultConst(centre) of src into
  // intt (num_q limbs) and the BConv of every dnum group i into dst[i].
  // ModUpGroups: ModUpBconv into modup + i * group_stride, then the column
  // pass (with_rows: and the row pass) of NTTForModUp for all groups in one
  // launch each. Own limbs of a group are left unwritten.
  // With src_mul, the ModUp input is the element-wise MontMul(src, src_mul)
  // (the Tensor's rx of HMult, formed on the fly).
  void ModUpBconv(word *const *dst, const DvConstView<word> &src,
                  word *intt, const word *src_mul = nullptr) const;
  void ModUpGroups(word *modup, long long group_stride,
                   const DvConstView<word> &src, word *intt,
                   bool with_rows, const word *src_mul = nullptr) const;
  // ModUpGroups (column passes only) of num_inputs (<= CHD_MAX_JOBS)
  // independent inputs of this level in one launch per phase: input i is
  // src + i * src_stride (num_q limbs), its group z goes to
  // modup + (i * NumGroups() + z) * group_stride, and intt holds
  // num_inputs * num_q limbs of scratch.
  void ModUpGroupsBatch(word *modup, long long group_stride, const word *src,
                        long long src_stride, int num_inputs,
                        word *intt) const;

  enum class Kind { ModDown, Rescale, ModDownAndRescale };
  // ModDownWorker for several polynomials at once: polynomial p of the
  // source starts at src + p * src_pstride (words, either sign: the
  // polynomials may sit in separate allocations), its result goes to
  // dst[p] (separate buffers allowed).
  // intt_rows: when given, the first pass of the INTT (stages 15..8) of the
  // INTT limbs is already there ([polynomial][limb] of the INTT limbs, as
  // the key accumulation leaves it), and only the second pass runs.
  void ModDownMulti(const std::vector<word *> &dst, const word *src,
                    long long src_pstride, Kind kind,
                    word *intt_rows = nullptr) const;
  // The source limbs a ModDown / ModDownAndRescale of this level transforms
  // back (its INTT limbs): [*first, *first + *count), contiguous. False when
  // they include terminal limbs (then they are not contiguous) or for
  // Rescale.
  bool ModDownInttRange(Kind kind, int *first, int *count) const;
  // words of workspace temporaries ModDownMulti takes for num_polys
  // polynomials (intt_rows_given: the first INTT pass is supplied)
  size_t ModDownScratchWords(Kind kind, int num_polys,
                             bool intt_rows_given) const;

 private:
  struct SwitchTable {       // one source set -> destination set
    DeviceVector<word> const1;   // (N prod_{j!=i} s_j)^-1 mod s_i
    DevBuf table;                // packed BConv table (chd_bconv_table_pack)
    // one source only: its table column, canonical per destination (the
    // NTT of the ModDown tail then forms the BConv itself)
    DeviceVector<word> bconv1;
    int src_len = 0, dst_len = 0;
  };
  // restore: destination primes [restore_lo, restore_hi) come back without
  // a source limb (BitPacker, ModSwitch.cu:320-370)
  void BuildSwitch(SwitchTable &st, const std::vector<word> &src,
                   const std::vector<word> &dst, int restore_lo = 0,
                   int restore_hi = 0) const;
  void ModDownWorker(DvView<word> &dst, const DvConstView<word> &src,
                     Kind kind) const;
  // source, destination and untransformed prime sets of a ModDown kind
  void ModDownShape(Kind kind, NPInfo *np_src, NPInfo *np_dst,
                    NPInfo *np_non_intt) const;
  const int level_;
  const int num_aux_;
  const int beta_;
  const int prime_offset_, first_group_, group_shift_;
  const Parameter<word> &param_;
  const NTTHandler<word> &ntt_;
  Workspace *ws_;
  DeviceVector<word> mod_up1_;
  std::vector<SwitchTable> mod_up_;
  SwitchTable mod_down_, rescale_, mod_down_rescale_;
  DeviceVector<word> inv_prime_prod_, rescale_inv_prime_prod_,
      mod_down_rescale_inv_prime_prod_;
  // BitPacker padding of the kept limbs (ModSwitch.cu:372-411); empty when
  // the rescale restores no prime (the padding is then the identity)
  DeviceVector<word> rescale_padding_, mod_down_rescale_padding_;
};

// CKKS encoder (include/core/Encode.h, src/core/Encode.cpp). Host arithmetic
// in IEEE double in the reference's operation order: the special IFFT with
// its twiddle indexing, division by the slot count, scaling, truncation
// toward zero and non-negative residues, then the device NTT with Montgomery
// conversion. The host part is compiled with -ffp-contract=off so no product
// and sum fuse: the residues are bit-identical to the reference's for every
// message it accepts. Decode inverts it through INTTAndMultConst, an exact
// CRT with a normalisation to (-Q/2, Q/2] and libtommath's conversion to
// double (the reference's default big-integer backend).
using Complex = std::complex<double>;
template <typename word>
class Encoder;
template <>
class Encoder<uint32_t> {
 public:
  using word = uint32_t;
  Encoder(const Parameter<word> &param, const NTTHandler<word> &ntt_handler);
  // host half only (SpecialIFFT / SpecialFFT / CoefficientResidues): no
  // device tables are needed, Encode / Decode / EncodeConstant throw
  explicit Encoder(const Parameter<word> &param);
  // Encode.cpp:23-43: the message is zero-padded to a power of two slots
  void Encode(Plaintext<word> &ptxt, int level, double scale,
              const std::vector<Complex> &message, int num_aux = 0) const;
  // Encode.cpp:45-82: aux primes are not supported, as in the reference
  void Decode(std::vector<Complex> &message, const Plaintext<word> &ptxt) const;
  // Encode.cpp:248-273: round(number * scale) truncated, per-prime Montgomery
  void EncodeConstant(Constant<word> &constant, int level, double scale,
                      double number, int num_aux = 0) const;
  Complex GetTwiddleFactor(int index) const { return twiddle_.at(index); }
  // ComplexVectorToPlaintext's host residues (before the NTT), [limb][N];
  // the message must already hold a power-of-two slot count
  std::vector<word> CoefficientResidues(int level, double scale,
                                        std::vector<Complex> data,
                                        int num_aux = 0) const;
  // Encode in two halves: the message zero-padded to a power of two slots,
  // and the device half (upload of CoefficientResidues' output, NTT with
  // Montgomery conversion). CoefficientResidues is const and reads only
  // immutable tables, so several threads may run it at once.
  static std::vector<Complex> PadToPowerOfTwo(
      const std::vector<Complex> &message);
  void EncodeResidues(Plaintext<word> &ptxt, int level, double scale,
                      int slots, const std::vector<word> &mx,
                      int num_aux = 0) const;
  void SpecialIFFT(std::vector<Complex> &data) const;
  void SpecialFFT(std::vector<Complex> &data) const;

 private:
  const Parameter<word> &param_;
  const NTTHandler<word> *ntt_handler_;
  const int m_;  // 2N
  std::vector<Complex> twiddle_;
};

template <typename word>
class Context;
template <>
class Context<uint32_t> {
 public:
  using word = uint32_t;
  using Dv = DeviceVector<word>;
  using Ct = Ciphertext<word>;
  using Evk = EvaluationKey<word>;
  static std::shared_ptr<Context<word>> Create(const Parameter<word> &param);

  // reference entry points (Context.h:302-423)
  void Mult(Ct &res, const Ct &a, const Ct &b) const;
  void HMult(Ct &res, const Ct &a, const Ct &b, const Evk &mult_key,
             bool rescale = true) const;
  void Relinearize(Ct &res, const Ct &a, const Evk &key) const;
  void RelinearizeRescale(Ct &res, const Ct &a, const Evk &key) const;
  void MultKey(Ct &res, const Ct &a, const Evk &key) const;
  void Rescale(Ct &res, const Ct &a) const;
  void HRot(Ct &res, const Ct &a, const Evk &rot_key, int rot_dist) const;
  void Permute(Ct &res, const Ct &a, int rot_dist) const;
  // Special-purpose key products for bootstrapping and hoisting
  // (Context.h:420-423, Context.cpp:609-712): the key switch without its
  // ModDown. accum gets the level's q primes plus alpha aux primes, a's
  // scale and slot count, and no rx; it may not be a (or a_orig).
  // PAccum of a caller-held ModUp: a_modup[g] is dnum group g of the ModUp
  // (ModSwitchHandler::ModUp's output, num_q + alpha limbs; groups holding
  // no limb of a_orig's level may be empty), multiplied by the key's group g
  // and summed over the extended basis.
  void MultKeyNoModDown(Ct &accum, const std::vector<Dv> &a_modup,
                        const Ct &a_orig, const Evk &key) const;
  // ModUp of a's rx (relinearisation) or of its ax (MultKey), the PAccum
  // above, then p_prod * (bx, ax) (or bx alone) added on the q limbs.
  // a may not carry aux primes.
  void MultKeyNoModDown(Ct &accum, const Ct &a, const Evk &key) const;

  // element-wise entry points (Context.h:95-300, Context.cpp:132-560,
  // 794-929); operands share the primes (and scale, where added)
  using Pt = Plaintext<word>;
  using Const = Constant<word>;
  void Copy(Ct &res, const Ct &a) const;
  void Add(Ct &res, const Ct &a, const Ct &b) const;
  void Add(Ct &res, const Ct &a, const Pt &b) const;
  void Add(Ct &res, const Ct &a, const Const &b) const;
  void Sub(Ct &res, const Ct &a, const Ct &b) const;
  void Sub(Ct &res, const Ct &a, const Pt &b) const;
  void Sub(Ct &res, const Ct &a, const Const &b) const;
  void Sub(Ct &res, const Pt &a, const Ct &b) const;
  void Sub(Ct &res, const Const &a, const Ct &b) const;
  void Neg(Ct &res, const Ct &a) const;
  void Mult(Ct &res, const Ct &a, const Pt &b) const;
  void Mult(Ct &res, const Ct &a, const Const &b) const;
  bool IsMultUnsafeCompatible(int level1, int level2) const;
  void MultUnsafe(Ct &res, const Ct &a, const Ct &b, int level = -1) const;
  void MultUnsafe(Ct &res, const Ct &a, const Pt &b, int level = -1) const;
  void MultUnsafe(Ct &res, const Ct &a, const Const &b, int level = -1) const;
  void PermuteConjugate(Ct &res, const Ct &a) const;
  void MultImaginaryUnit(Ct &res, const Ct &a) const;
  void HConj(Ct &res, const Ct &a, const Evk &conj_key) const;
  void HRotAdd(Ct &res, const Ct &a, const Ct &b, const Evk &rot_key,
               int rot_dist) const;
  void HConjAdd(Ct &res, const Ct &a, const Ct &b, const Evk &conj_key) const;
  // res += a * b on res's primes (Context.cpp:873-915)
  void MadUnsafe(Ct &res, const Ct &a, const Const &b) const;
  // multiplication by the encoded constant 1 at the level's scale, then
  // Rescale, down to target_level (Context.cpp:917-929)
  void LevelDown(Ct &res, const Ct &a, int target_level) const;

  // view-level core used by the C++ API above and by the C-ABI
  struct CtRef {           // polynomials of num_q limbs (rx optional)
    word *bx = nullptr, *ax = nullptr, *rx = nullptr;
  };
  struct CtCRef {
    const word *bx = nullptr, *ax = nullptr, *rx = nullptr;
  };
  struct EvkRef {          // beta pairs of evk_limbs limbs each
    std::vector<const word *> bx, ax;
    NPInfo np;
  };
  void TensorV(int level, CtRef res, CtCRef a, CtCRef b) const;
  // accum (b, a) of num_q + alpha limbs = KS of d, plus p_prod * (cb, ca)
  void KeyMultNoModDownV(int level, word *acc_b, word *acc_a, const word *d,
                         const word *cb, const word *ca,
                         const EvkRef &key) const;
  // the same for HMult with the Tensor fused in: d = rx, (cb, ca) = (bx, ax)
  // of a x b, formed inside the ModUp and accumulation kernels
  void KeyMultTensorV(int level, word *acc_b, word *acc_a, CtCRef a, CtCRef b,
                      const EvkRef &key) const;
  void HMultV(int level, CtRef res, CtCRef a, CtCRef b, const EvkRef &key,
              bool rescale) const;
  void RescaleV(int level, CtRef res, CtCRef a) const;
  void MultKeyV(int level, CtRef res, CtCRef a, const EvkRef &key) const;
  void PermuteV(int level, CtRef res, CtCRef a, int galois_amount) const;
  // scratch arena of this context (sized for HMult / HRot at the top level)
  Workspace *GetWorkspace() const { return ws_.get(); }
  // peak words of workspace temporaries of HMultV / MultKeyV at a level
  size_t KeySwitchScratchWords(int level, bool rescale) const;
  // MultKeyNoModDown of an extended-basis accumulator (Context.cpp:609-643,
  // as the giant step of Hoist.cu:939-957 uses it): the ModUp of d (q limbs,
  // level's prime count), multiplied by the key and summed over the dnum
  // groups, plus add_b (q + alpha limbs) on the b part.
  void KeyMultExtV(int level, word *acc_b, word *acc_a, const word *d,
                   const word *add_b, const EvkRef &key) const;
  // the PAccum of MultKeyNoModDown(accum, a_modup, a_orig, key) on views:
  // modup[g] for g < GetBeta() of the level's ModSwitchHandler, each
  // num_q + alpha limbs (unread, and may be null, for groups before its
  // FirstGroup()); acc_b / acc_a get num_q + alpha limbs
  void KeyMultModUpV(int level, word *acc_b, word *acc_a,
                     const word *const *modup, const EvkRef &key) const;
  // KeyMultExtV of num (<= CHD_MAX_JOBS) independent inputs at one level,
  // each with its own key: input i is d + i * d_stride, its add_b is
  // add_b + i * add_stride and its result goes to (acc_b[i], acc_a[i]).
  // One launch per phase for all of them (the giant steps of Hoist.cu:
  // 895-957 are independent until their permuted sum).
  void KeyMultExtBatchV(int level, int num, word *const *acc_b,
                        word *const *acc_a, const word *d, long long d_stride,
                        const word *add_b, long long add_stride,
                        const EvkRef *const *keys) const;
  static EvkRef RefOfKey(const Evk &k);
  DvConstView<word> PProd(const NPInfo &np) const { return GetPProd(np); }

  const Parameter<word> &param_;
  ElementWiseHandler<word> elem_handler_;
  NTTHandler<word> ntt_handler_;
  std::vector<ModSwitchHandler<word>> mod_switch_handlers_;
  Encoder<word> encoder_;

 private:
  explicit Context(const Parameter<word> &param);
  DvConstView<word> GetPProd(const NPInfo &np) const;
  void KeyAccumulate(int level, word *acc_b, word *acc_a, const word *d,
                     const word *cb, const word *ca, const CtCRef *ta,
                     const CtCRef *tb, const EvkRef &key,
                     const word *add_b = nullptr, word *intt_b = nullptr,
                     word *intt_a = nullptr, int intt_lo = 0) const;
  void KeySwitchDown(int level, CtRef res, const word *d, const word *cb,
                     const word *ca, const CtCRef *ta, const CtCRef *tb,
                     const EvkRef &key, bool rescale) const;
  DeviceVector<word> p_prod_;
  std::unique_ptr<Workspace> ws_;
  // EncodeConstant(1.0) at each level's default scale, for LevelDown
  std::vector<Constant<word>> level_down_consts_;
};

template <typename word>
using ConstContextPtr = std::shared_ptr<const Context<word>>;

// Baby-step / giant-step evaluation with double hoisting
// (include/extension/Hoist.h, src/extension/Hoist.cu), the non-min_ks
// optimized path: res = Rescale(sum_g Rot_g(sum_b pt[g][b] * Rot_b(input))).
//
// Two constructors, as in the reference: from complex messages, which are
// encoded at (pt_level, alpha aux primes) with pt_scale (Hoist.cu:131-177,
// including the bs/gs swap of single-giant-step maps), or from plaintexts
// already encoded in that form (mx_ holds num_q(pt_level) + alpha limbs in
// the NTT domain). A giant step 0 must be present when there are other giant
// steps and more than one baby step (the reference's optimized path reads
// its accumulator unconditionally).
//
// Maps whose giant steps all hold only baby step 0 (the swapped maps; the
// reference's bs == 1 path, Hoist.cu:715-797) multiply the key-switched
// input by pt_g before the automorphism g. Permute only moves NTT-domain
// residues, so Permute_g(x pt_g) = Permute_g(x) Permute_g(pt_g) exactly; such
// a map is evaluated as the single giant step 0 with baby steps g and
// plaintexts Permute_g(pt_g), prepared once here: the same residues, the
// same rotation keys.
template <typename word>
class HoistHandler;
template <>
class HoistHandler<uint32_t> {
 public:
  using word = uint32_t;
  using Ct = Ciphertext<word>;
  using Pt = Plaintext<word>;
  using PtMap = std::map<int, std::map<int, Pt>>;  // gs -> bs -> plaintext
  using Message = std::vector<Complex>;
  using PlainHoistMap = std::map<int, std::map<int, Message>>;
  HoistHandler(ConstContextPtr<word> context, const PlainHoistMap &hoist_map,
               int pt_level, double pt_scale, bool suppress_bs_swap = false);
  HoistHandler(ConstContextPtr<word> context, PtMap &&encoded, int pt_level,
               double pt_scale);
  HoistHandler(const HoistHandler &) = delete;
  HoistHandler &operator=(const HoistHandler &) = delete;
  HoistHandler(HoistHandler &&) = default;

  // rotation keys Evaluate needs (Hoist.cu:978-1004); with min_ks the two
  // strides of the baby- and giant-step sequences
  void AddRequiredRotations(EvkRequest &req, bool min_ks = false) const;
  std::set<int> RequiredRotations(bool min_ks = false) const;
  // min_ks (Hoist.cu:517-566): baby steps by repeated HRot with the
  // baby-step stride, giant steps Horner-style with the giant-step stride,
  // so only two rotation keys are needed
  void Evaluate(ConstContextPtr<word> context, Ct &res, const Ct &input,
                const EvkMap<word> &evk_map, bool min_ks = false) const;
  void EvaluateBabyStep(ConstContextPtr<word> context, std::map<int, Ct> &bs,
                        const Ct &input, const EvkMap<word> &evk_map,
                        bool min_ks = false) const;
  void EvaluateGiantStep(ConstContextPtr<word> context, Ct &res,
                         const std::map<int, Ct> &bs,
                         const EvkMap<word> &evk_map,
                         bool min_ks = false) const;

  // the same with keys looked up by rotation index through a callback
  // (used by the C-ABI, whose keys are raw device pointers)
  using KeyLookup = std::function<Context<word>::EvkRef(int)>;
  void BabyStep(const Context<word> &ctx, std::map<int, Ct> &bs,
                const Ct &input, const KeyLookup &key,
                bool min_ks = false) const;
  void GiantStep(const Context<word> &ctx, Ct &res,
                 const std::map<int, Ct> &bs, const KeyLookup &key,
                 bool min_ks = false) const;

 private:
  int pt_level_;
  double pt_scale_;
  std::pair<int, int> CheckStrideMinKS() const;
  void MinKSBabyStep(const Context<word> &ctx, std::map<int, Ct> &bs,
                     const Ct &input, const KeyLookup &key_of) const;
  void MinKSGiantStep(const Context<word> &ctx, Ct &res,
                      const std::map<int, Ct> &bs,
                      const KeyLookup &key_of) const;
  static PtMap EncodeMap(const Context<word> &context,
                         const PlainHoistMap &hoist_map, int pt_level,
                         double pt_scale, bool suppress_bs_swap);
  PtMap pt_map_;
  std::set<int> bs_indices_;
  std::vector<int> gs_indices_;
  bool gs_only_ = false;  // a giant-step-only map, evaluated converted
  // wide giant-step accumulation (more than CHD_GS_MAX_GS giant steps, at
  // most CHD_GS_WIDE_GS, at most CHD_GS_MAX_BS baby steps): device table of
  // plaintext addresses [giant step][baby step] in gs_indices_ x
  // bs_indices_ order, padded to wide_gs_ rows and wide_bs_ (a multiple of
  // 4) columns; absent pairs and padding point at zero_pt_, padding rows
  // write to dummy_out_ (never read). Built once at construction.
  int wide_gs_ = 0, wide_bs_ = 0;
  DevBuf pt_table_, zero_pt_, dummy_out_;
  // tiled copy of the first tiled_rows_ giant steps' plaintexts
  // (chd_k_gs_pack_tiled), read by the wide accumulation; 0 rows: none
  int tiled_rows_ = 0;
  DevBuf pt_tiled_;
};

// Square matrix by its generalised diagonals (include/extension/
// StripedMatrix.h, src/extension/StripedMatrix.cpp): diagonal i holds
// M[j][(j + i) % width] at j.
class StripedMatrix : public std::map<int, std::vector<Complex>> {
 public:
  using Base = std::map<int, std::vector<Complex>>;
  explicit StripedMatrix(int height = 0, int width = 0)
      : height_(height), width_(width) {}
  int GetHeight() const { return height_; }
  int GetWidth() const { return width_; }
  int GetNumDiag() const { return static_cast<int>(size()); }
  static StripedMatrix Mult(const StripedMatrix &a, const StripedMatrix &b);
  static StripedMatrix Mult(const StripedMatrix &a, const Complex b);

 private:
  int height_, width_;
};

// Matrix-vector product by BSGS over a HoistHandler
// (include/extension/LinearTransform.h, src/extension/LinearTransform.cpp).
template <typename word>
class LinearTransform;
template <>
class LinearTransform<uint32_t> {
 public:
  using word = uint32_t;
  using Ct = Ciphertext<word>;
  LinearTransform(ConstContextPtr<word> context, const StripedMatrix &matrix,
                  int pt_level, double pt_scale, int bs, int gs = 1,
                  int pre_rotation = 0, int additional_pt_rot = 0);
  bool IsUsingBSGS() const { return bs_ > 1 && gs_ > 1; }
  int GetBS() const { return bs_; }
  int GetGS() const { return gs_; }
  int GetPreRotationAmount() const { return pre_rotation_; }
  void AddRequiredRotations(EvkRequest &req, bool min_ks = false) const {
    hoist_.AddRequiredRotations(req, min_ks);
  }
  void Evaluate(ConstContextPtr<word> context, Ct &res, const Ct &input,
                const EvkMap<word> &evk_map, bool min_ks = false) const {
    hoist_.Evaluate(context, res, input, evk_map, min_ks);
  }
  const HoistHandler<word> &GetHoistHandler() const { return hoist_; }
  // the reference's hoist map for a matrix (LinearTransform.cpp:40-72)
  static HoistHandler<word>::PlainHoistMap ConstructPlainHoistMap(
      const StripedMatrix &matrix, int bs, int gs, int pre_rotation,
      int additional_pt_rot);

 private:
  static int DetermineStride(const StripedMatrix &matrix, int bs, int gs,
                             int pre_rotation);
  int bs_, gs_, pre_rotation_;
  HoistHandler<word> hoist_;
};

}  // namespace cheddar
