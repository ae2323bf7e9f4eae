// Element-wise ElementWiseHandler ops and the Context entry points built on
// them (src/core/ElementWise.cu:674-920, 1673-1706; src/core/Context.cpp:
// 10-60, 132-560, 794-929). Scale, slot count and rx follow the reference
// call by call; every op runs as one chd_k_elementwise launch per call.
#include <algorithm>
#include <climits>
#include <cmath>

#include "cheddar.h"
#include "cheddar_amd.h"
#include "prime_math.h"

namespace cheddar {

namespace {

void K(int status) {
  if (status != 0) throw Error(chd_last_error());
}

chd_limb_map LevelMap(const Parameter<uint32_t> &param, const NPInfo &np) {
  chd_limb_map m{};
  m.num_q = np.GetNumQ();
  m.skip_lo = INT_MAX;
  m.tab_off = param.TerLeft(np);
  m.tab_gap = param.MainLeft(np);
  return m;
}

}  // namespace

// ------------------------------------------------- ElementWiseHandler ops --
void ElementWiseHandler<uint32_t>::Elementwise(int op, Views &dst,
                                               const NPInfo &np,
                                               const CViews &src1,
                                               const CViews *src2,
                                               const DvConstView<word> *cst)
    const {
  const int n = param_.degree_;
  const int num_poly = static_cast<int>(dst.size());
  AssertTrue(num_poly > 0 && num_poly <= CHD_MAX_POLY,
             "ElementWise: Invalid number of polynomials");
  AssertTrue(static_cast<int>(src1.size()) == num_poly,
             "ElementWise: Incompatible dst/src size");
  const int q_size = np.GetNumQ() * n;
  const int aux_size = np.num_aux_ * n;
  for (const auto &d : dst)
    AssertTrue(d.QSize() == q_size && d.TotalSize() == q_size + aux_size,
               "ElementWise: dst size mismatch");
  auto gap = [&](const DvConstView<word> &v) {
    AssertTrue(v.QSize() >= q_size && v.QSize() % n == 0 &&
                   v.TotalSize() >= v.QSize() + aux_size,
               "ElementWise: src too small for its limbs");
    return (v.QSize() - q_size) / n;
  };
  chd_ew_args a{};
  a.op = op;
  a.num_poly = num_poly;
  a.a_gap = gap(src1[0]);
  for (int p = 0; p < num_poly; p++) {
    AssertTrue(gap(src1[p]) == a.a_gap, "ElementWise: src layout mismatch");
    a.dst[p] = dst[p].data();
    a.a[p] = src1[p].data();
  }
  if (src2 != nullptr) {
    const int nb = op == CHD_EW_PMULT ? 1 : num_poly;
    AssertTrue(static_cast<int>(src2->size()) == nb,
               "ElementWise: Incompatible dst/src size");
    a.b_gap = gap((*src2)[0]);
    for (int p = 0; p < nb; p++) {
      AssertTrue(gap((*src2)[p]) == a.b_gap,
                 "ElementWise: src layout mismatch");
      a.b[p] = (*src2)[p].data();
    }
  }
  if (cst != nullptr) {
    AssertTrue(cst->QSize() >= np.GetNumQ() &&
                   cst->TotalSize() >= cst->QSize() + np.num_aux_,
               "ElementWise: constant too small for its limbs");
    a.cst = cst->data();
    a.cst_gap = cst->QSize() - np.GetNumQ();
  }
  const chd_limb_map m = LevelMap(param_, np);
  K(chd_k_elementwise(&ntt_.Tables(), &m, &a, np.GetNumTotal(),
                      CurrentStream()));
}

void ElementWiseHandler<uint32_t>::Add(Views &dst, const NPInfo &np,
                                       const CViews &src1,
                                       const CViews &src2) const {
  Elementwise(CHD_EW_ADD, dst, np, src1, &src2, nullptr);
}
void ElementWiseHandler<uint32_t>::Sub(Views &dst, const NPInfo &np,
                                       const CViews &src1,
                                       const CViews &src2) const {
  Elementwise(CHD_EW_SUB, dst, np, src1, &src2, nullptr);
}
void ElementWiseHandler<uint32_t>::Neg(Views &dst, const NPInfo &np,
                                       const CViews &src1) const {
  Elementwise(CHD_EW_NEG, dst, np, src1, nullptr, nullptr);
}
void ElementWiseHandler<uint32_t>::Mult(Views &dst, const NPInfo &np,
                                        const CViews &src1,
                                        const CViews &src2) const {
  Elementwise(CHD_EW_MULT, dst, np, src1, &src2, nullptr);
}
void ElementWiseHandler<uint32_t>::PMult(Views &dst, const NPInfo &np,
                                         const CViews &src1,
                                         const DvConstView<word> &src2) const {
  const CViews b{src2};
  Elementwise(CHD_EW_PMULT, dst, np, src1, &b, nullptr);
}
void ElementWiseHandler<uint32_t>::AddConst(
    Views &dst, const NPInfo &np, const CViews &src1,
    const DvConstView<word> &src_const) const {
  Elementwise(CHD_EW_ADD_CONST, dst, np, src1, nullptr, &src_const);
}
void ElementWiseHandler<uint32_t>::SubConst(
    Views &dst, const NPInfo &np, const CViews &src1,
    const DvConstView<word> &src_const) const {
  Elementwise(CHD_EW_SUB_CONST, dst, np, src1, nullptr, &src_const);
}
void ElementWiseHandler<uint32_t>::SubOppositeConst(
    Views &dst, const NPInfo &np, const CViews &src1,
    const DvConstView<word> &src_const) const {
  Elementwise(CHD_EW_SUB_OPP_CONST, dst, np, src1, nullptr, &src_const);
}
void ElementWiseHandler<uint32_t>::MultConst(
    Views &dst, const NPInfo &np, const CViews &src1,
    const DvConstView<word> &src_const) const {
  Elementwise(CHD_EW_MULT_CONST, dst, np, src1, nullptr, &src_const);
}
// ElementWise.cu:626-660: by +-ToMont(psi^(N/2)) of each limb (the table the
// reference reads at twiddle_factors_ + 1, NTT.cu:1302-1310). The reference
// kernel reads aux limbs of that table without the aux gap; here aux limbs
// use their own primes' entries.
void ElementWiseHandler<uint32_t>::MultImaginaryUnit(
    Views &dst, const NPInfo &np, const CViews &src1) const {
  Elementwise(CHD_EW_MULT_I, dst, np, src1, nullptr, nullptr);
}
void ElementWiseHandler<uint32_t>::Copy(Views &dst, const NPInfo &np,
                                        const CViews &src1) const {
  Elementwise(CHD_EW_COPY, dst, np, src1, nullptr, nullptr);
}

// ---------------------------------------------------- Context entry points
namespace {

using Ct = Ciphertext<uint32_t>;
using word = uint32_t;

// Context.cpp:10-30
void MatchResultWith(Ct &res, const Ct &a, bool rx) {
  if (rx) {
    res.ModifyNP(a.GetNP());
    res.PrepareRx();
  } else {
    res.RemoveRx();
    res.ModifyNP(a.GetNP());
  }
}

// Context.cpp:54-60
void AssertSameScale(double s1, double s2) {
  AssertTrue(std::fabs(s1 - s2) < 1e-12 * s1, "Scale mismatch");
}

// views of a polynomial of np's shape starting front limbs in
DvView<word> PolyView(DeviceVector<word> &v, const NPInfo &np, int n,
                      int front = 0) {
  return DvView<word>(v.data() + static_cast<size_t>(front) * n,
                      static_cast<int>(v.size()) - front * n,
                      np.num_aux_ * n);
}
DvConstView<word> PolyCView(const DeviceVector<word> &v, const NPInfo &np,
                            int n, int front = 0) {
  return DvConstView<word>(v.data() + static_cast<size_t>(front) * n,
                           static_cast<int>(v.size()) - front * n,
                           np.num_aux_ * n);
}

}  // namespace

// Context.cpp:132-144
void Context<uint32_t>::Copy(Ct &res, const Ct &a) const {
  if (&res == &a) return;
  MatchResultWith(res, a, a.HasRx());
  res.SetNumSlots(a.GetNumSlots());
  res.SetScale(a.GetScale());
  const NPInfo np = a.GetNP();
  const int n = param_.degree_;
  std::vector<DvView<word>> d{PolyView(res.bx_, np, n),
                              PolyView(res.ax_, np, n)};
  std::vector<DvConstView<word>> s{PolyCView(a.bx_, np, n),
                                   PolyCView(a.ax_, np, n)};
  if (a.HasRx()) {
    d.push_back(PolyView(res.rx_, np, n));
    s.push_back(PolyCView(a.rx_, np, n));
  }
  elem_handler_.Copy(d, np, s);
}

// Context.cpp:146-168 (Ct + Ct) and 205-229 (Ct - Ct)
namespace {
template <typename F, typename G>
void AddSubCt(const Context<word> &ctx, Ct &res, const Ct &a, const Ct &b,
              F op, G rx_only_b) {
  AssertTrue(a.GetNP() == b.GetNP(), "NP mismatch");
  AssertSameScale(a.GetScale(), b.GetScale());
  const bool rx_both = a.HasRx() && b.HasRx();
  const NPInfo np = a.GetNP();
  const int n = ctx.param_.degree_;
  // b's rx may be lost when res aliases b and rx must be copied or negated
  const bool keep_b_rx = !rx_both && b.HasRx() && &res == &b;
  DeviceVector<word> b_rx;
  if (keep_b_rx) {
    b_rx.resize(b.rx_.size());
    HipCheck(hipMemcpyAsync(b_rx.data(), b.rx_.data(),
                            b.rx_.size() * sizeof(word),
                            hipMemcpyDeviceToDevice, CurrentStream()),
             "hipMemcpyAsync");
  }
  const double scale = a.GetScale();
  const int slots = std::max(a.GetNumSlots(), b.GetNumSlots());
  const bool a_rx = a.HasRx(), b_has_rx = b.HasRx();
  const DeviceVector<word> *a_rx_src = a_rx ? &a.rx_ : nullptr;
  MatchResultWith(res, a, a_rx || b_has_rx);
  res.SetNumSlots(slots);
  res.SetScale(scale);
  std::vector<DvView<word>> d{PolyView(res.bx_, np, n),
                              PolyView(res.ax_, np, n)};
  std::vector<DvConstView<word>> x{PolyCView(a.bx_, np, n),
                                   PolyCView(a.ax_, np, n)};
  std::vector<DvConstView<word>> y{PolyCView(b.bx_, np, n),
                                   PolyCView(b.ax_, np, n)};
  if (rx_both) {
    d.push_back(PolyView(res.rx_, np, n));
    x.push_back(PolyCView(a.rx_, np, n));
    y.push_back(PolyCView(b.rx_, np, n));
  }
  op(d, np, x, y);
  if (rx_both) return;
  std::vector<DvView<word>> r{PolyView(res.rx_, np, n)};
  if (a_rx) {
    if (a_rx_src != &res.rx_)
      ctx.elem_handler_.Copy(r, np, {PolyCView(*a_rx_src, np, n)});
  } else if (b_has_rx) {
    rx_only_b(r, np, keep_b_rx ? PolyCView(b_rx, np, n)
                               : PolyCView(b.rx_, np, n));
  }
}
}  // namespace

void Context<uint32_t>::Add(Ct &res, const Ct &a, const Ct &b) const {
  AddSubCt(
      *this, res, a, b,
      [&](auto &d, const NPInfo &np, const auto &x, const auto &y) {
        elem_handler_.Add(d, np, x, y);
      },
      [&](std::vector<DvView<word>> &r, const NPInfo &np,
          const DvConstView<word> &brx) { elem_handler_.Copy(r, np, {brx}); });
}

void Context<uint32_t>::Sub(Ct &res, const Ct &a, const Ct &b) const {
  AddSubCt(
      *this, res, a, b,
      [&](auto &d, const NPInfo &np, const auto &x, const auto &y) {
        elem_handler_.Sub(d, np, x, y);
      },
      [&](std::vector<DvView<word>> &r, const NPInfo &np,
          const DvConstView<word> &brx) { elem_handler_.Neg(r, np, {brx}); });
}

// Context.cpp:171-203, 231-263: b applies to bx only; ax (and rx) copied
namespace {
template <typename F>
void CtWithB(const Context<word> &ctx, Ct &res, const Ct &a, const NPInfo &bnp,
             double bscale, int bslots, F op) {
  AssertTrue(a.GetNP() == bnp, "NP mismatch");
  AssertSameScale(a.GetScale(), bscale);
  const NPInfo np = a.GetNP();
  const int n = ctx.param_.degree_;
  const int slots = std::max(a.GetNumSlots(), bslots);
  const double scale = a.GetScale();
  MatchResultWith(res, a, a.HasRx());
  res.SetNumSlots(slots);
  res.SetScale(scale);
  std::vector<DvView<word>> d{PolyView(res.bx_, np, n)};
  op(d, np, PolyCView(a.bx_, np, n));
  if (&res == &a) return;
  std::vector<DvView<word>> r{PolyView(res.ax_, np, n)};
  std::vector<DvConstView<word>> s{PolyCView(a.ax_, np, n)};
  if (a.HasRx()) {
    r.push_back(PolyView(res.rx_, np, n));
    s.push_back(PolyCView(a.rx_, np, n));
  }
  ctx.elem_handler_.Copy(r, np, s);
}
}  // namespace

void Context<uint32_t>::Add(Ct &res, const Ct &a, const Pt &b) const {
  CtWithB(*this, res, a, b.GetNP(), b.GetScale(), b.GetNumSlots(),
          [&](auto &d, const NPInfo &np, const DvConstView<word> &x) {
            elem_handler_.Add(d, np, {x},
                              {PolyCView(b.mx_, np, param_.degree_)});
          });
}

void Context<uint32_t>::Add(Ct &res, const Ct &a, const Const &b) const {
  CtWithB(*this, res, a, b.GetNP(), b.GetScale(), 0,
          [&](auto &d, const NPInfo &np, const DvConstView<word> &x) {
            elem_handler_.AddConst(
                d, np, {x},
                DvConstView<word>(b.cx_.data(),
                                  static_cast<int>(b.cx_.size()),
                                  np.num_aux_));
          });
}

void Context<uint32_t>::Sub(Ct &res, const Ct &a, const Pt &b) const {
  CtWithB(*this, res, a, b.GetNP(), b.GetScale(), b.GetNumSlots(),
          [&](auto &d, const NPInfo &np, const DvConstView<word> &x) {
            elem_handler_.Sub(d, np, {x},
                              {PolyCView(b.mx_, np, param_.degree_)});
          });
}

void Context<uint32_t>::Sub(Ct &res, const Ct &a, const Const &b) const {
  CtWithB(*this, res, a, b.GetNP(), b.GetScale(), 0,
          [&](auto &d, const NPInfo &np, const DvConstView<word> &x) {
            elem_handler_.SubConst(
                d, np, {x},
                DvConstView<word>(b.cx_.data(),
                                  static_cast<int>(b.cx_.size()),
                                  np.num_aux_));
          });
}

// Context.cpp:265-304: bx = a - b.bx, ax (and rx) negated
namespace {
template <typename F>
void BMinusCt(const Context<word> &ctx, Ct &res, const NPInfo &anp,
              double ascale, int aslots, const Ct &b, F op) {
  AssertTrue(anp == b.GetNP(), "NP mismatch");
  AssertSameScale(ascale, b.GetScale());
  const NPInfo np = b.GetNP();
  const int n = ctx.param_.degree_;
  const int slots = std::max(aslots, b.GetNumSlots());
  MatchResultWith(res, b, b.HasRx());
  res.SetNumSlots(slots);
  res.SetScale(ascale);
  std::vector<DvView<word>> d{PolyView(res.bx_, np, n)};
  op(d, np, PolyCView(b.bx_, np, n));
  std::vector<DvView<word>> r{PolyView(res.ax_, np, n)};
  std::vector<DvConstView<word>> s{PolyCView(b.ax_, np, n)};
  if (b.HasRx()) {
    r.push_back(PolyView(res.rx_, np, n));
    s.push_back(PolyCView(b.rx_, np, n));
  }
  ctx.elem_handler_.Neg(r, np, s);
}
}  // namespace

void Context<uint32_t>::Sub(Ct &res, const Pt &a, const Ct &b) const {
  BMinusCt(*this, res, a.GetNP(), a.GetScale(), a.GetNumSlots(), b,
           [&](auto &d, const NPInfo &np, const DvConstView<word> &x) {
             elem_handler_.Sub(d, np, {PolyCView(a.mx_, np, param_.degree_)},
                               {x});
           });
}

void Context<uint32_t>::Sub(Ct &res, const Const &a, const Ct &b) const {
  BMinusCt(*this, res, a.GetNP(), a.GetScale(), 0, b,
           [&](auto &d, const NPInfo &np, const DvConstView<word> &x) {
             elem_handler_.SubOppositeConst(
                 d, np, {x},
                 DvConstView<word>(a.cx_.data(),
                                   static_cast<int>(a.cx_.size()),
                                   np.num_aux_));
           });
}

// Context.cpp:306-315
void Context<uint32_t>::Neg(Ct &res, const Ct &a) const {
  const NPInfo np = a.GetNP();
  const int n = param_.degree_;
  const int slots = a.GetNumSlots();
  const double scale = a.GetScale();
  MatchResultWith(res, a, a.HasRx());
  res.SetNumSlots(slots);
  res.SetScale(scale);
  std::vector<DvView<word>> d{PolyView(res.bx_, np, n),
                              PolyView(res.ax_, np, n)};
  std::vector<DvConstView<word>> s{PolyCView(a.bx_, np, n),
                                   PolyCView(a.ax_, np, n)};
  if (a.HasRx()) {
    d.push_back(PolyView(res.rx_, np, n));
    s.push_back(PolyCView(a.rx_, np, n));
  }
  elem_handler_.Neg(d, np, s);
}

// Context.cpp:333-355 (and MultUnsafe, 414-500): every polynomial of a times
// b, on the primes of `level`, skipping the leading terminal limbs a or b
// has beyond them
namespace {
template <typename F>
void MultByB(const Context<word> &ctx, Ct &res, const Ct &a,
             const NPInfo &res_np, const NPInfo &bnp, double bscale,
             int bslots, F op) {
  const NPInfo anp = a.GetNP();
  const int n = ctx.param_.degree_;
  const int a_front = anp.num_ter_ - res_np.num_ter_;
  const int b_front = bnp.num_ter_ - res_np.num_ter_;
  if (&res == &a && !(anp == res_np)) {
    Ct tmp;
    MultByB(ctx, tmp, a, res_np, bnp, bscale, bslots, op);
    res = std::move(tmp);
    return;
  }
  const int slots = std::max(a.GetNumSlots(), bslots);
  const double scale = a.GetScale() * bscale;
  if (a.HasRx()) {
    res.ModifyNP(res_np);
    res.PrepareRx();
  } else {
    res.RemoveRx();
    res.ModifyNP(res_np);
  }
  res.SetNumSlots(slots);
  res.SetScale(scale);
  std::vector<DvView<word>> d{PolyView(res.bx_, res_np, n),
                              PolyView(res.ax_, res_np, n)};
  std::vector<DvConstView<word>> s{PolyCView(a.bx_, anp, n, a_front),
                                   PolyCView(a.ax_, anp, n, a_front)};
  if (a.HasRx()) {
    d.push_back(PolyView(res.rx_, res_np, n));
    s.push_back(PolyCView(a.rx_, anp, n, a_front));
  }
  op(d, res_np, s, b_front);
}
}  // namespace

void Context<uint32_t>::Mult(Ct &res, const Ct &a, const Pt &b) const {
  AssertTrue(a.GetNP() == b.GetNP(), "NP mismatch");
  MultUnsafe(res, a, b, param_.NPToLevel(NPInfo(a.GetNP().num_main_,
                                                a.GetNP().num_ter_, 0)));
}

void Context<uint32_t>::Mult(Ct &res, const Ct &a, const Const &b) const {
  AssertTrue(a.GetNP() == b.GetNP(), "NP mismatch");
  MultUnsafe(res, a, b, param_.NPToLevel(NPInfo(a.GetNP().num_main_,
                                                a.GetNP().num_ter_, 0)));
}

// Context.cpp:357-367
bool Context<uint32_t>::IsMultUnsafeCompatible(int level1, int level2) const {
  if (level1 == level2) return true;
  const NPInfo lo = param_.LevelToNP(std::min(level1, level2));
  const NPInfo hi = param_.LevelToNP(std::max(level1, level2));
  return lo.IsSubsetOf(hi);
}

void Context<uint32_t>::MultUnsafe(Ct &res, const Ct &a, const Pt &b,
                                   int level) const {
  const NPInfo anp = a.GetNP(), bnp = b.GetNP();
  if (level == -1)
    level = std::min(param_.NPToLevel(NPInfo(anp.num_main_, anp.num_ter_, 0)),
                     param_.NPToLevel(NPInfo(bnp.num_main_, bnp.num_ter_, 0)));
  const NPInfo res_np =
      param_.LevelToNP(level, std::min(anp.num_aux_, bnp.num_aux_));
  AssertTrue(res_np.IsSubsetOf(anp) && res_np.IsSubsetOf(bnp),
             "Incompatible levels for MultUnsafe Ct x Pt");
  MultByB(*this, res, a, res_np, bnp, b.GetScale(), b.GetNumSlots(),
          [&](auto &d, const NPInfo &np, const auto &s, int b_front) {
            elem_handler_.PMult(d, np, s,
                                PolyCView(b.mx_, bnp, param_.degree_, b_front));
          });
}

void Context<uint32_t>::MultUnsafe(Ct &res, const Ct &a, const Const &b,
                                   int level) const {
  const NPInfo anp = a.GetNP(), bnp = b.GetNP();
  if (level == -1)
    level = std::min(param_.NPToLevel(NPInfo(anp.num_main_, anp.num_ter_, 0)),
                     param_.NPToLevel(NPInfo(bnp.num_main_, bnp.num_ter_, 0)));
  const NPInfo res_np =
      param_.LevelToNP(level, std::min(anp.num_aux_, bnp.num_aux_));
  AssertTrue(res_np.IsSubsetOf(anp) && res_np.IsSubsetOf(bnp),
             "Incompatible levels for MultUnsafe Ct x Const");
  MultByB(*this, res, a, res_np, bnp, b.GetScale(), 0,
          [&](auto &d, const NPInfo &np, const auto &s, int b_front) {
            elem_handler_.MultConst(
                d, np, s,
                DvConstView<word>(b.cx_.data() + b_front,
                                  static_cast<int>(b.cx_.size()) - b_front,
                                  bnp.num_aux_));
          });
}

// Context.cpp:370-412: the Tensor of a and b on the primes of `level`
void Context<uint32_t>::MultUnsafe(Ct &res, const Ct &a, const Ct &b,
                                   int level) const {
  AssertTrue(!a.HasRx() && !b.HasRx(),
             "Relinearization required before MultUnsafe Ct x Ct");
  const NPInfo anp = a.GetNP(), bnp = b.GetNP();
  AssertTrue(anp.num_aux_ == 0 && bnp.num_aux_ == 0,
             "MultUnsafe Ct x Ct should be only used for ciphertexts without "
             "aux primes");
  const int al = param_.NPToLevel(anp), bl = param_.NPToLevel(bnp);
  if (level == -1) level = std::min(al, bl);
  if ((&res == &a && al != level) || (&res == &b && bl != level)) {
    Ct tmp;
    MultUnsafe(tmp, a, b, level);
    res = std::move(tmp);
    return;
  }
  const NPInfo res_np = param_.LevelToNP(level, 0);
  AssertTrue(res_np.IsSubsetOf(anp) && res_np.IsSubsetOf(bnp),
             "Incompatible levels for MultUnsafe Ct x Ct");
  const int n = param_.degree_;
  const int af = anp.num_ter_ - res_np.num_ter_;
  const int bf = bnp.num_ter_ - res_np.num_ter_;
  const int slots = std::max(a.GetNumSlots(), b.GetNumSlots());
  const double scale = a.GetScale() * b.GetScale();
  // a Ct operand that res aliases is read before it is resized (same
  // level, so ModifyNP keeps its buffers)
  res.ModifyNP(res_np);
  res.PrepareRx();
  res.SetNumSlots(slots);
  res.SetScale(scale);
  std::vector<DvView<word>> d{PolyView(res.bx_, res_np, n),
                              PolyView(res.ax_, res_np, n),
                              PolyView(res.rx_, res_np, n)};
  elem_handler_.Tensor(d, res_np,
                       {PolyCView(a.bx_, anp, n, af),
                        PolyCView(a.ax_, anp, n, af)},
                       {PolyCView(b.bx_, bnp, n, bf),
                        PolyCView(b.ax_, bnp, n, bf)});
}

// Context.cpp:530-548: permutation by the Galois factor 2N - 1
void Context<uint32_t>::PermuteConjugate(Ct &res, const Ct &a) const {
  if (&res == &a) {
    Ct tmp;
    PermuteConjugate(tmp, a);
    res = std::move(tmp);
    return;
  }
  const NPInfo np = a.GetNP();
  const int n = param_.degree_;
  MatchResultWith(res, a, a.HasRx());
  res.SetNumSlots(a.GetNumSlots());
  res.SetScale(a.GetScale());
  std::vector<DvView<word>> d{PolyView(res.bx_, np, n),
                              PolyView(res.ax_, np, n)};
  std::vector<DvConstView<word>> s{PolyCView(a.bx_, np, n),
                                   PolyCView(a.ax_, np, n)};
  if (a.HasRx()) {
    d.push_back(PolyView(res.rx_, np, n));
    s.push_back(PolyCView(a.rx_, np, n));
  }
  elem_handler_.Permute(d, np, -1, s);
}

// Context.cpp:550-560
void Context<uint32_t>::MultImaginaryUnit(Ct &res, const Ct &a) const {
  const NPInfo np = a.GetNP();
  const int n = param_.degree_;
  const int slots = a.GetNumSlots();
  const double scale = a.GetScale();
  MatchResultWith(res, a, a.HasRx());
  res.SetNumSlots(slots);
  res.SetScale(scale);
  std::vector<DvView<word>> d{PolyView(res.bx_, np, n),
                              PolyView(res.ax_, np, n)};
  std::vector<DvConstView<word>> s{PolyCView(a.bx_, np, n),
                                   PolyCView(a.ax_, np, n)};
  if (a.HasRx()) {
    d.push_back(PolyView(res.rx_, np, n));
    s.push_back(PolyCView(a.rx_, np, n));
  }
  elem_handler_.MultImaginaryUnit(d, np, s);
}

// Context.cpp:794-799
void Context<uint32_t>::HConj(Ct &res, const Ct &a, const Evk &conj_key) const {
  Ct tmp;
  MultKey(tmp, a, conj_key);
  PermuteConjugate(res, tmp);
}

// Context.cpp:801-861: Permute(MultKey(a)) + b in one PermuteAccum
namespace {
void RotAdd(const Context<word> &ctx, Ct &res, const Ct &a, const Ct &b,
            const Context<word>::Evk &key, int amount) {
  Ct tmp;
  ctx.MultKey(tmp, a, key);
  const NPInfo np = a.GetNP();
  const int n = ctx.param_.degree_;
  DeviceVector<word> b_rx;
  if (b.HasRx()) {  // b's rx is kept; copy it first in case res aliases b
    b_rx.resize(b.rx_.size());
    HipCheck(hipMemcpyAsync(b_rx.data(), b.rx_.data(),
                            b.rx_.size() * sizeof(word),
                            hipMemcpyDeviceToDevice, CurrentStream()),
             "hipMemcpyAsync");
  }
  Ct bcopy;
  const Ct *bp = &b;
  if (&res == &b) {  // PermuteAccum reads b whole after others wrote res
    ctx.Copy(bcopy, b);
    bp = &bcopy;
  }
  if (b.HasRx()) {
    res.ModifyNP(np);
    res.PrepareRx();
  } else {
    res.RemoveRx();
    res.ModifyNP(np);
  }
  std::vector<DvView<word>> d{PolyView(res.bx_, np, n),
                              PolyView(res.ax_, np, n)};
  ctx.elem_handler_.PermuteAccum(
      d, np, {amount},
      {{PolyCView(tmp.bx_, np, n), PolyCView(tmp.ax_, np, n)},
       {PolyCView(bp->bx_, np, n), PolyCView(bp->ax_, np, n)}});
  if (b.HasRx()) {
    std::vector<DvView<word>> r{PolyView(res.rx_, np, n)};
    ctx.elem_handler_.Copy(r, np, {PolyCView(b_rx, np, n)});
  }
}
}  // namespace

void Context<uint32_t>::HRotAdd(Ct &res, const Ct &a, const Ct &b,
                                const Evk &rot_key, int rot_dist) const {
  AssertTrue(a.GetNP() == b.GetNP(), "NP mismatch");
  AssertSameScale(a.GetScale(), b.GetScale());
  const int slots = std::max(a.GetNumSlots(), b.GetNumSlots());
  int r = rot_dist % slots;
  if (r < 0) r += slots;
  const double scale = a.GetScale();
  if (r == 0) {
    Add(res, a, b);
  } else {
    RotAdd(*this, res, a, b, rot_key, r);
  }
  res.SetNumSlots(slots);
  res.SetScale(scale);
}

void Context<uint32_t>::HConjAdd(Ct &res, const Ct &a, const Ct &b,
                                 const Evk &conj_key) const {
  AssertTrue(a.GetNP() == b.GetNP(), "NP mismatch");
  AssertSameScale(a.GetScale(), b.GetScale());
  const int slots = std::max(a.GetNumSlots(), b.GetNumSlots());
  const double scale = a.GetScale();
  RotAdd(*this, res, a, b, conj_key, -1);
  res.SetNumSlots(slots);
  res.SetScale(scale);
}

// Context.cpp:873-915: res += a * b (CAccum) on res's primes
void Context<uint32_t>::MadUnsafe(Ct &res, const Ct &a, const Const &b) const {
  const NPInfo anp = a.GetNP(), bnp = b.GetNP(), rnp = res.GetNP();
  AssertTrue(rnp.IsSubsetOf(anp) && rnp.IsSubsetOf(bnp),
             "Incompatible levels for MultUnsafe Ct x Const");
  AssertTrue(rnp.num_aux_ == 0 && anp.num_aux_ == 0,
             "MadUnsafe should be only used for q primes");
  AssertTrue(res.GetNumSlots() == a.GetNumSlots(),
             "MadUnsafe should be only used for the same number of slots");
  AssertSameScale(res.GetScale(), a.GetScale() * b.GetScale());
  if (a.HasRx() && !res.HasRx()) {
    // PrepareRx leaves rx undefined, as in the reference; clear it so the
    // accumulation starts from zero
    res.PrepareRx();
    K(chd_k_zero(res.rx_.data(), static_cast<long long>(res.rx_.size()),
                 CurrentStream()));
  }
  const int n = param_.degree_;
  const int af = anp.num_ter_ - rnp.num_ter_;
  const int bf = bnp.num_ter_ - rnp.num_ter_;
  std::vector<DvView<word>> d{PolyView(res.bx_, rnp, n),
                              PolyView(res.ax_, rnp, n)};
  std::vector<DvConstView<word>> s{PolyCView(a.bx_, anp, n, af),
                                   PolyCView(a.ax_, anp, n, af)};
  std::vector<DvConstView<word>> r{PolyCView(res.bx_, rnp, n),
                                   PolyCView(res.ax_, rnp, n)};
  if (a.HasRx()) {
    d.push_back(PolyView(res.rx_, rnp, n));
    s.push_back(PolyCView(a.rx_, anp, n, af));
    r.push_back(PolyCView(res.rx_, rnp, n));
  }
  elem_handler_.CAccum(
      d, rnp, {s, r},
      {DvConstView<word>(b.cx_.data() + bf,
                         static_cast<int>(b.cx_.size()) - bf, 0)});
}

// Context.cpp:917-929 with the constants of 102-107
void Context<uint32_t>::LevelDown(Ct &res, const Ct &a,
                                  int target_level) const {
  const int level = param_.NPToLevel(a.GetNP());
  AssertTrue(level >= target_level && target_level >= 0,
             "Invalid target level for LevelDown");
  AssertTrue(level <= param_.default_encryption_level_,
             "LevelDown: no level-down constant above the default "
             "encryption level");
  if (level == target_level) {
    Copy(res, a);
    return;
  }
  Ct mult_tmp, next;
  const Ct *prev = &a;
  for (int i = level; i > target_level; i--) {
    Mult(mult_tmp, *prev, level_down_consts_.at(i));
    Rescale(next, mult_tmp);
    prev = &next;
  }
  Copy(res, *prev);
}

}  // namespace cheddar
