// C++ drop-in API test: the reference's own call shapes (Parameter,
// Context::Create, Ciphertext / EvaluationKey containers, Context::HMult /
// HRot / MultKey / Rescale / Mult + Relinearize(Rescale), and the public
// handler members) on config-4 sizes, checked bit-exactly against the CPU
// oracle (oracle/oracle.h), which this test links as its checker.
//
// Mirrors the structure of the reference's unittest/BasicTest.cpp: build a
// parameter set, run one operation per test, compare. Prints one line per
// test; exit status 0 only if every test passes. Needs a HIP device.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "cheddar.h"
#include "oracle.h"

using namespace cheddar;
using word = uint32_t;
using Ct = Ciphertext<word>;
using Evk = EvaluationKey<word>;

namespace {

constexpr int kLogN = 16;
constexpr size_t kN = size_t{1} << kLogN;

uint64_t g_state = 0xC0FFEE04ull;
uint64_t next64() {  // splitmix64
  uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

std::vector<word> primes(int bits, int count) {
  std::vector<word> r;
  const uint64_t step = 1u << 17;
  uint64_t q = ((uint64_t{1} << bits) - 1) / step * step + 1;
  auto is_prime = [](uint64_t n) {
    for (uint64_t d = 2; d * d <= n; d++)
      if (n % d == 0) return false;
    return true;
  };
  while (static_cast<int>(r.size()) < count) {
    if (is_prime(q)) r.push_back(static_cast<word>(q));
    q -= step;
  }
  return r;
}

// uniform residues, limb i under chain[i]
std::vector<word> uniform(const std::vector<word> &chain, int limbs) {
  std::vector<word> v(static_cast<size_t>(limbs) * kN);
  for (int l = 0; l < limbs; l++)
    for (size_t n = 0; n < kN; n++) v[l * kN + n] = next64() % chain[l];
  return v;
}

void upload(word *dst, const std::vector<word> &h) {
  HipCheck(hipMemcpy(dst, h.data(), h.size() * sizeof(word),
                     hipMemcpyHostToDevice),
           "hipMemcpy");
}
std::vector<word> download(const word *src, size_t words) {
  std::vector<word> h(words);
  HipCheck(hipDeviceSynchronize(), "hipDeviceSynchronize");
  HipCheck(hipMemcpy(h.data(), src, words * sizeof(word),
                     hipMemcpyDeviceToHost),
           "hipMemcpy");
  return h;
}

int g_fail = 0;
void check(const std::string &name, bool ok) {
  std::printf("%s %s\n", ok ? "PASS" : "FAIL", name.c_str());
  std::fflush(stdout);
  if (!ok) g_fail++;
}
bool same(const std::vector<word> &a, const std::vector<word> &b) {
  return a.size() == b.size() &&
         std::memcmp(a.data(), b.data(), a.size() * sizeof(word)) == 0;
}

}  // namespace

int main() {
  const int L = 24, alpha = 8;
  const std::vector<word> main_p = primes(30, L), aux_p = primes(31, alpha);
  std::vector<std::pair<int, int>> levels;
  for (int i = 1; i <= L; i++) levels.emplace_back(i, 0);
  // Parameter.h:42-47 argument order
  Parameter<word> param(kLogN, 0x1p30, L - 1, levels, main_p, aux_p);
  auto ctx = Context<word>::Create(param);
  orc_set_threads(8);

  const NPInfo np = param.LevelToNP(L - 1);
  const NPInfo np_key = param.LevelToNP(param.max_level_, alpha);
  const int beta = param.dnum_;
  const size_t qw = static_cast<size_t>(L) * kN;
  const size_t kw = static_cast<size_t>(L + alpha) * kN;
  std::vector<word> chain_k(main_p);
  chain_k.insert(chain_k.end(), aux_p.begin(), aux_p.end());

  // two ciphertexts and a key of beta groups (UserInterface.cu:522-541 shape)
  Ct a(np), b(np);
  const std::vector<word> hb1 = uniform(main_p, L), ha1 = uniform(main_p, L);
  const std::vector<word> hb2 = uniform(main_p, L), ha2 = uniform(main_p, L);
  upload(a.bx_.data(), hb1);
  upload(a.ax_.data(), ha1);
  upload(b.bx_.data(), hb2);
  upload(b.ax_.data(), ha2);
  a.SetScale(0x1p30);
  b.SetScale(0x1p30);
  Evk key(np_key, beta);
  std::vector<word> kb(beta * kw), ka(beta * kw);
  for (int g = 0; g < beta; g++) {
    const std::vector<word> x = uniform(chain_k, L + alpha);
    const std::vector<word> y = uniform(chain_k, L + alpha);
    std::copy(x.begin(), x.end(), kb.begin() + g * kw);
    std::copy(y.begin(), y.end(), ka.begin() + g * kw);
    upload(key.bx_[g].data(), x);
    upload(key.ax_[g].data(), y);
  }

  // oracle results
  std::vector<word> wb((L) * kN), wa((L) * kN), wbr((L - 1) * kN),
      war((L - 1) * kN);
  orc_hmult(wbr.data(), war.data(), hb1.data(), ha1.data(), hb2.data(),
            ha2.data(), kb.data(), ka.data(), L, L, main_p.data(),
            aux_p.data(), alpha, kLogN, 1);
  orc_hmult(wb.data(), wa.data(), hb1.data(), ha1.data(), hb2.data(),
            ha2.data(), kb.data(), ka.data(), L, L, main_p.data(),
            aux_p.data(), alpha, kLogN, 0);

  // Context::HMult with merged rescale (Context.cpp:862-871)
  {
    Ct res;
    ctx->HMult(res, a, b, key, true);
    check("HMult(rescale=true) level and scale",
          res.GetNP() == param.LevelToNP(L - 2) &&
              res.GetScale() == 0x1p60 / param.GetRescalePrimeProd(L - 1));
    check("HMult(rescale=true) bx", same(download(res.bx_.data(), (L - 1) * kN), wbr));
    check("HMult(rescale=true) ax", same(download(res.ax_.data(), (L - 1) * kN), war));
  }
  // HMult without rescale, then Rescale (Context.cpp:739-774)
  {
    Ct res, res2;
    ctx->HMult(res, a, b, key, false);
    check("HMult(rescale=false) bx", same(download(res.bx_.data(), qw), wb));
    check("HMult(rescale=false) ax", same(download(res.ax_.data(), qw), wa));
    ctx->Rescale(res2, res);
    std::vector<word> rb((L - 1) * kN), ra((L - 1) * kN);
    orc_rescale(rb.data(), wb.data(), L, main_p.data(), 1, kLogN);
    orc_rescale(ra.data(), wa.data(), L, main_p.data(), 1, kLogN);
    check("Rescale bx", same(download(res2.bx_.data(), (L - 1) * kN), rb));
    check("Rescale ax", same(download(res2.ax_.data(), (L - 1) * kN), ra));
  }
  // Mult (tensor with rx) then Relinearize / RelinearizeRescale
  {
    Ct t, r1, r2;
    ctx->Mult(t, a, b);
    check("Mult keeps rx", t.HasRx());
    ctx->Relinearize(r1, t, key);
    check("Mult + Relinearize == HMult(false)",
          same(download(r1.bx_.data(), qw), wb) &&
              same(download(r1.ax_.data(), qw), wa));
    ctx->RelinearizeRescale(r2, t, key);
    check("Mult + RelinearizeRescale == HMult(true)",
          same(download(r2.bx_.data(), (L - 1) * kN), wbr) &&
              same(download(r2.ax_.data(), (L - 1) * kN), war));
  }
  // in place: res aliases the first input (Context.cpp:867)
  {
    Ct c(np);
    upload(c.bx_.data(), hb1);
    upload(c.ax_.data(), ha1);
    c.SetScale(0x1p30);
    ctx->HMult(c, c, b, key, true);
    check("HMult in place",
          same(download(c.bx_.data(), (L - 1) * kN), wbr) &&
              same(download(c.ax_.data(), (L - 1) * kN), war));
  }
  // the device pool behind DeviceVector (MemoryPool.cpp:5-35): the
  // reference's bins for this parameter set, and result ciphertexts made per
  // call (the reference's usage) served from it once warm
  {
    const std::vector<size_t> want_bins = {
        512,    2048,    8192,    32768,   131072,  262144,
        524288, 1048576, 2097152, 4194304, 6291456, 8388608};
    check("memory pool bins", MemoryPool::Current().Bins() == want_bins);
    bool ok = true;
    size_t warm = 0;
    const size_t reuses0 = MemoryPool::Current().GetStats().reuses;
    for (int i = 0; i < 20; i++) {
      Ct res;
      ctx->HMult(res, a, b, key, true);
      ok = ok && same(download(res.bx_.data(), (L - 1) * kN), wbr) &&
           same(download(res.ax_.data(), (L - 1) * kN), war);
      if (i == 1) warm = MemoryPool::Current().GetStats().device_allocations;
    }
    const MemoryPool::Stats st = MemoryPool::Current().GetStats();
    check("HMult with a new result ciphertext per call", ok);
    check("per-call results come from the pool, no device allocation",
          st.device_allocations == warm && st.reuses - reuses0 >= 38);
  }
  // DeviceVector::resize keeps the leading words (device_uvector::resize),
  // ZeroExtend appends zeros (DeviceVector.cpp:75-85)
  {
    const std::vector<word> head(hb1.begin(), hb1.begin() + 4 * kN);
    DeviceVector<word> v(4 * kN);
    upload(v.data(), head);
    const word *p0 = v.data();
    v.resize(2 * kN);
    check("DeviceVector shrink keeps memory and data",
          v.data() == p0 &&
              same(download(v.data(), 2 * kN),
                   std::vector<word>(head.begin(), head.begin() + 2 * kN)));
    v.resize(6 * kN);
    check("DeviceVector growth keeps the leading words",
          v.size() == 6 * kN &&
              same(download(v.data(), 2 * kN),
                   std::vector<word>(head.begin(), head.begin() + 2 * kN)));
    v.ZeroExtend(kN);
    const std::vector<word> tail = download(v.data() + 6 * kN, kN);
    check("DeviceVector ZeroExtend",
          v.size() == 7 * kN &&
              same(tail, std::vector<word>(kN, 0)));
    HostVector<word> back;
    DeviceVector<word> w;
    CopyHostToDevice(w, head);
    CopyDeviceToHost(back, w);
    HipCheck(hipDeviceSynchronize(), "hipDeviceSynchronize");
    check("CopyHostToDevice / CopyDeviceToHost", same(back, head));
  }
  // MultKey and HRot (Context.cpp:584-607, 776-791)
  {
    Ct mk, rot;
    ctx->MultKey(mk, a, key);
    std::vector<word> mb(qw), ma(qw);
    orc_mult_key(mb.data(), ma.data(), hb1.data(), ha1.data(), kb.data(),
                 ka.data(), L, L, main_p.data(), aux_p.data(), alpha, kLogN);
    check("MultKey", same(download(mk.bx_.data(), qw), mb) &&
                         same(download(mk.ax_.data(), qw), ma));
    ctx->HRot(rot, a, key, 5);
    std::vector<word> hrb(qw), hra(qw);
    orc_hrot(hrb.data(), hra.data(), hb1.data(), ha1.data(), kb.data(),
             ka.data(), L, L, main_p.data(), aux_p.data(), alpha, kLogN, 5);
    check("HRot(5)", same(download(rot.bx_.data(), qw), hrb) &&
                         same(download(rot.ax_.data(), qw), hra));
  }
  // Context::MultKeyNoModDown, both overloads (Context.h:420-423,
  // Context.cpp:609-712), shaped as the reference's hoisting calls them
  // (Hoist.cu:676, 771, 849): a caller-held ModUp of a.ax, a.ax itself (the
  // MultKey branch) and a tensor with rx (the relinearisation branch),
  // against orc_mod_up + orc_paccum (+ orc_caccum)
  {
    std::vector<word> pp(L);
    orc_p_prod(pp.data(), main_p.data(), L, aux_p.data(), alpha);
    auto key_mult = [&](const std::vector<word> &d, std::vector<word> &ob,
                        std::vector<word> &oa) {
      std::vector<word> up(static_cast<size_t>(beta) * kw);
      orc_mod_up(up.data(), d.data(), L, main_p.data(), aux_p.data(), alpha,
                 kLogN);
      ob.assign(kw, 0);
      oa.assign(kw, 0);
      orc_paccum(ob.data(), oa.data(), up.data(), beta, kb.data(), ka.data(),
                 L, alpha, L, chain_k.data(), kLogN);
    };
    const NPInfo np_acc(L, 0, alpha);
    std::vector<word> pb, pa;
    key_mult(ha1, pb, pa);

    // (accum, a_modup, a_orig, key): the PAccum of a ModUp the caller holds
    const auto &ms = ctx->mod_switch_handlers_[L - 1];
    std::vector<DeviceVector<word>> up(ms.GetBeta());
    std::vector<DvView<word>> upv;
    for (auto &u : up) {
      u.resize(kw);
      upv.push_back(u.View(alpha * static_cast<int>(kN)));
    }
    ms.ModUp(upv, a.ax_.ConstView());
    Ct acc;
    ctx->MultKeyNoModDown(acc, up, a, key);
    check("MultKeyNoModDown(accum, a_modup, a_orig, key)",
          acc.GetNP() == np_acc && !acc.HasRx() &&
              acc.GetScale() == a.GetScale() &&
              same(download(acc.bx_.data(), kw), pb) &&
              same(download(acc.ax_.data(), kw), pa));

    // (accum, a, key) without rx: ModUp(ax), PAccum, P * bx on the q limbs
    std::vector<word> wb2 = pb;
    orc_caccum(wb2.data(), hb1.data(), pp.data(), L, main_p.data(), kLogN);
    ctx->MultKeyNoModDown(acc, a, key);
    check("MultKeyNoModDown(accum, a, key), MultKey branch",
          acc.GetNP() == np_acc && same(download(acc.bx_.data(), kw), wb2) &&
              same(download(acc.ax_.data(), kw), pa));

    // (accum, a, key) with rx: ModUp(rx), PAccum, P * (bx, ax)
    Ct t;
    ctx->Mult(t, a, b);
    std::vector<word> tb(qw), ta(qw), tr(qw), rb, ra;
    orc_tensor(tb.data(), ta.data(), tr.data(), hb1.data(), ha1.data(),
               hb2.data(), ha2.data(), L, main_p.data(), kLogN);
    key_mult(tr, rb, ra);
    orc_caccum(rb.data(), tb.data(), pp.data(), L, main_p.data(), kLogN);
    orc_caccum(ra.data(), ta.data(), pp.data(), L, main_p.data(), kLogN);
    ctx->MultKeyNoModDown(acc, t, key);
    check("MultKeyNoModDown(accum, a, key), relinearisation branch",
          acc.GetNP() == np_acc && acc.GetScale() == t.GetScale() &&
              same(download(acc.bx_.data(), kw), rb) &&
              same(download(acc.ax_.data(), kw), ra));
    // ModDown of that accumulator is Relinearize (Context.cpp:584-607 with
    // 645-712)
    DeviceVector<word> md(qw);
    DvView<word> mdv = md.View();
    ms.ModDown(mdv, acc.bx_.ConstView(alpha * static_cast<int>(kN)));
    check("ModDown(MultKeyNoModDown(a * b)) == HMult(rescale=false)",
          same(download(md.data(), qw), wb));

    // the reference's asserts: no in-place, no aux primes in a
    bool in_place = false, with_aux = false;
    try {
      ctx->MultKeyNoModDown(t, t, key);
    } catch (const Error &) {
      in_place = true;
    }
    try {
      Ct acc2;
      ctx->MultKeyNoModDown(acc2, acc, key);
    } catch (const Error &) {
      with_aux = true;
    }
    check("MultKeyNoModDown rejects in-place and aux-prime inputs",
          in_place && with_aux);
  }
  // public handler members (Context.h:83-92), used directly by extensions
  {
    DeviceVector<word> y(qw);
    DvView<word> yv = y.View();
    ctx->ntt_handler_.NTT(yv, np, a.bx_.ConstView(), false);
    std::vector<word> want = hb1;
    orc_ntt_batch(want.data(), L, kLogN, main_p.data(), 0);
    check("ntt_handler_.NTT", same(download(y.data(), qw), want));
    DeviceVector<word> z(qw);
    DvView<word> zv = z.View();
    ctx->ntt_handler_.INTT(zv, np, y.ConstView(), false);
    check("ntt_handler_.INTT round trip", same(download(z.data(), qw), hb1));

    const auto &ms = ctx->mod_switch_handlers_[L - 1];
    std::vector<DeviceVector<word>> up(ms.GetBeta());
    std::vector<DvView<word>> upv;
    for (auto &u : up) {
      u.resize(kw);
      upv.push_back(u.View(alpha * static_cast<int>(kN)));
    }
    ms.ModUp(upv, a.ax_.ConstView());
    std::vector<word> wup(static_cast<size_t>(ms.GetBeta()) * kw);
    orc_mod_up(wup.data(), ha1.data(), L, main_p.data(), aux_p.data(), alpha,
               kLogN);
    bool ok = true;
    for (int g = 0; g < ms.GetBeta(); g++)
      ok = ok && same(download(up[g].data(), kw),
                      std::vector<word>(wup.begin() + g * kw,
                                        wup.begin() + (g + 1) * kw));
    check("mod_switch_handlers_[level].ModUp", ok);
  }
  // elem_handler_ seams the reference's extensions call directly
  // (Hoist.cu:484, UserInterface.cu:185): PAccum with polynomial commons
  // (ElementWise.cu:1396-1435) over aux-extended polynomials, more
  // accumulands than one launch takes plus an extra addend; CAccum with
  // per-limb constants; Tensor; Permute
  {
    const NPInfo npx = param.LevelToNP(L - 1, alpha);
    const int tl = npx.GetNumTotal();
    const size_t tw = static_cast<size_t>(tl) * kN;
    const std::vector<word> &chain = chain_k;  // main then aux primes
    const int num_acc = 11;                    // two launches of <= 8
    std::vector<std::vector<word>> hct(num_acc + 1), hcm(num_acc), hct2(num_acc + 1);
    std::vector<DeviceVector<word>> dct, dcm, dct2;
    auto to_dev = [&](const std::vector<word> &h) {
      DeviceVector<word> d(h.size());
      upload(d.data(), h);
      return d;
    };
    for (int j = 0; j <= num_acc; j++) {
      hct[j] = uniform(chain, tl);
      hct2[j] = uniform(chain, tl);
      dct.push_back(to_dev(hct[j]));
      dct2.push_back(to_dev(hct2[j]));
      if (j < num_acc) {
        hcm[j] = uniform(chain, tl);
        dcm.push_back(to_dev(hcm[j]));
      }
    }
    const int aux_words = alpha * static_cast<int>(kN);
    std::vector<std::vector<DvConstView<word>>> srcs;
    std::vector<DvConstView<word>> commons;
    for (int j = 0; j <= num_acc; j++)
      srcs.push_back({dct[j].ConstView(aux_words), dct2[j].ConstView(aux_words)});
    for (int j = 0; j < num_acc; j++) commons.push_back(dcm[j].ConstView(aux_words));
    DeviceVector<word> o1(tw), o2(tw);
    std::vector<DvView<word>> out{o1.View(aux_words), o2.View(aux_words)};
    ctx->elem_handler_.PAccum(out, npx, srcs, commons);
    bool ok = true;
    for (int p = 0; p < 2 && ok; p++) {
      const std::vector<word> got = download(p ? o2.data() : o1.data(), tw);
      const auto &hs = p ? hct2 : hct;
      for (int l = 0; l < tl && ok; l++)
        for (size_t c = 0; c < kN && ok; c++) {
          const size_t i = l * kN + c;
          uint64_t acc = hs[num_acc][i];
          for (int j = 0; j < num_acc; j++)
            acc += orc_mont_mul(hs[j][i], hcm[j][i], chain[l]);
          ok = got[i] == acc % chain[l];
        }
    }
    check("elem_handler_.PAccum (polynomial commons, 11 + extra addend)", ok);

    // CAccum: one Montgomery constant per limb (a Constant's cx_)
    const int num_c = 3;
    std::vector<std::vector<word>> hc(num_c);
    std::vector<DeviceVector<word>> dc;
    std::vector<DvConstView<word>> cviews;
    std::vector<std::vector<DvConstView<word>>> csrcs;
    for (int j = 0; j < num_c; j++) {
      hc[j].resize(tl);
      for (int l = 0; l < tl; l++) hc[j][l] = next64() % chain[l];
      dc.push_back(to_dev(hc[j]));
      cviews.push_back(dc[j].ConstView(alpha));
      csrcs.push_back({dct[j].ConstView(aux_words)});
    }
    std::vector<DvView<word>> cout{o1.View(aux_words)};
    ctx->elem_handler_.CAccum(cout, npx, csrcs, cviews);
    ok = true;
    {
      const std::vector<word> got = download(o1.data(), tw);
      for (int l = 0; l < tl && ok; l++)
        for (size_t c = 0; c < kN && ok; c++) {
          const size_t i = l * kN + c;
          uint64_t acc = 0;
          for (int j = 0; j < num_c; j++)
            acc += orc_mont_mul(hct[j][i], hc[j][l], chain[l]);
          ok = got[i] == acc % chain[l];
        }
    }
    check("elem_handler_.CAccum (per-limb constants)", ok);

    // Tensor (ElementWise.cu:921-953) and Permute (ElementWise.cu:966-999)
    DeviceVector<word> tb(qw), ta(qw), tr(qw);
    std::vector<DvView<word>> tdst{tb.View(), ta.View(), tr.View()};
    ctx->elem_handler_.Tensor(tdst, np, {a.bx_.ConstView(), a.ax_.ConstView()},
                              {b.bx_.ConstView(), b.ax_.ConstView()});
    std::vector<word> wtb(qw), wta(qw), wtr(qw);
    orc_tensor(wtb.data(), wta.data(), wtr.data(), hb1.data(), ha1.data(),
               hb2.data(), ha2.data(), L, main_p.data(), kLogN);
    check("elem_handler_.Tensor", same(download(tb.data(), qw), wtb) &&
                                      same(download(ta.data(), qw), wta) &&
                                      same(download(tr.data(), qw), wtr));
    std::vector<DvView<word>> pdst{tb.View(), ta.View()};
    ctx->elem_handler_.Permute(pdst, np, 77,
                               {a.bx_.ConstView(), a.ax_.ConstView()});
    std::vector<word> wpb(qw), wpa(qw);
    const uint32_t gal = ctx->elem_handler_.PermuteAmountToGaloisFactor(77);
    orc_permute(wpb.data(), hb1.data(), L, kLogN, gal);
    orc_permute(wpa.data(), ha1.data(), L, kLogN, gal);
    check("elem_handler_.Permute(77)",
          gal == orc_galois_factor(77, kLogN) &&
              same(download(tb.data(), qw), wpb) &&
              same(download(ta.data(), qw), wpa));
  }
  // encoder member (Context.h:88): Encode / Decode round trip within the
  // reference's EncodeDecode tolerance (Testbed.h:93), EncodeConstant
  {
    std::vector<Complex> msg(1 << 12);
    for (auto &m : msg)
      m = Complex((next64() % 2001) / 1000.0 - 1.0,
                  (next64() % 2001) / 1000.0 - 1.0);
    Plaintext<word> pt;
    ctx->encoder_.Encode(pt, L - 1, 0x1p30, msg);
    std::vector<Complex> back;
    ctx->encoder_.Decode(back, pt);
    double err = 0;
    for (size_t i = 0; i < msg.size(); i++)
      err = std::max(err, std::abs(back[i] - msg[i]));
    check("Encoder Encode/Decode round trip",
          pt.GetNumSlots() == (1 << 12) && pt.GetNP() == np && err < 1e-3);
    Constant<word> c;
    ctx->encoder_.EncodeConstant(c, 3, 0x1p20, -1.5);
    std::vector<word> cx = download(c.cx_.data(), c.cx_.size());
    bool ok = cx.size() == 4;
    for (int i = 0; i < 4 && ok; i++) {
      const uint64_t p = main_p[i];
      const uint64_t v = (p - (uint64_t{3} << 19) % p) % p;  // -1.5 * 2^20
      ok = cx[i] == (v << 32) % p;
    }
    check("Encoder EncodeConstant", ok);
  }
  // EvkRequest keeps the highest level per rotation (EvkRequest.cpp:7-17)
  {
    EvkRequest req;
    req.AddRequest(3, 5);
    req.AddRequest(3, 2);
    req.AddRequest(7, 1);
    req.AddRequest(3, 9);
    check("EvkRequest", req.size() == 2 && req.at(3) == 9 && req.at(7) == 1);
  }
  // StripedMatrix::Mult against the dense product (StripedMatrix.cpp:17-36)
  {
    const int w = 8;
    StripedMatrix a(w, w), b(w, w);
    for (int i : {0, 1, 5}) {
      a[i].resize(w);
      for (auto &v : a[i]) v = Complex(int(next64() % 7) - 3, int(next64() % 5) - 2);
    }
    for (int i : {2, 3}) {
      b[i].resize(w);
      for (auto &v : b[i]) v = Complex(int(next64() % 7) - 3, int(next64() % 5) - 2);
    }
    auto dense = [](const StripedMatrix &m) {
      std::vector<Complex> d(w * w);
      for (const auto &[i, diag] : m)
        for (int j = 0; j < w; j++) d[j * w + (j + i) % w] += diag[j];
      return d;
    };
    const std::vector<Complex> da = dense(a), db = dense(b);
    const std::vector<Complex> dc = dense(StripedMatrix::Mult(a, b));
    bool ok = true;
    for (int r = 0; r < w; r++)
      for (int c2 = 0; c2 < w; c2++) {
        Complex s = 0;
        for (int k = 0; k < w; k++) s += da[r * w + k] * db[k * w + c2];
        ok = ok && std::abs(s - dc[r * w + c2]) < 1e-12;
      }
    const std::vector<Complex> ds =
        dense(StripedMatrix::Mult(a, Complex(0.0, 2.0)));
    for (int k = 0; k < w * w; k++)
      ok = ok && std::abs(ds[k] - da[k] * Complex(0.0, 2.0)) < 1e-12;
    check("StripedMatrix::Mult", ok);
    // LinearTransform's hoist map (LinearTransform.cpp:40-72): diagonal 5 of
    // a bs = 2 transform lands at giant step 4, baby step 1, rotated right
    // by 4
    StripedMatrix m(w, w);
    for (int i : {0, 1, 2, 5}) {
      m[i].resize(w);
      for (int j = 0; j < w; j++) m[i][j] = Complex(10 * i + j, 0);
    }
    const auto map = LinearTransform<word>::ConstructPlainHoistMap(m, 2, 3, 0, 0);
    ok = map.size() == 3 && map.at(0).size() == 2 && map.at(2).size() == 1 &&
         map.at(4).size() == 1 && map.at(4).count(1) == 1;
    for (int j = 0; ok && j < w; j++)
      ok = map.at(4).at(1)[(j + 4) % w] == Complex(50 + j, 0);
    check("LinearTransform::ConstructPlainHoistMap", ok);
  }
  // element-wise Context ops (Context.cpp:132-315, 333-412, 530-560,
  // 794-929) against host modular arithmetic, the oracle's key switch and
  // permutation, and the encoder (decode of the b polynomial of a
  // ciphertext whose a polynomial is zero)
  {
    auto lanes = [&](const std::vector<word> &x, const std::vector<word> &y,
                     int limbs, auto f) {
      std::vector<word> r(static_cast<size_t>(limbs) * kN);
      for (int l = 0; l < limbs; l++)
        for (size_t n = 0; n < kN; n++)
          r[l * kN + n] = f(x[l * kN + n], y.empty() ? 0 : y[l * kN + n],
                            static_cast<uint64_t>(main_p[l]), l);
      return r;
    };
    auto add = [](uint64_t x, uint64_t y, uint64_t p, int) {
      return static_cast<word>((x + y) % p);
    };
    auto sub = [](uint64_t x, uint64_t y, uint64_t p, int) {
      return static_cast<word>((x + p - y) % p);
    };
    auto neg = [](uint64_t x, uint64_t, uint64_t p, int) {
      return static_cast<word>((p - x) % p);
    };
    auto mul = [](uint64_t x, uint64_t y, uint64_t p, int) {
      return orc_mont_mul(static_cast<word>(x), static_cast<word>(y),
                          static_cast<word>(p));
    };
    const std::vector<word> none;
    auto bx_of = [&](const Ct &c) {
      return download(c.bx_.data(), static_cast<size_t>(c.GetNP().GetNumQ()) * kN);
    };
    auto ax_of = [&](const Ct &c) {
      return download(c.ax_.data(), static_cast<size_t>(c.GetNP().GetNumQ()) * kN);
    };
    Ct r;
    ctx->Add(r, a, b);
    check("Context::Add(ct, ct)", same(bx_of(r), lanes(hb1, hb2, L, add)) &&
                                      same(ax_of(r), lanes(ha1, ha2, L, add)) &&
                                      r.GetScale() == 0x1p30 && !r.HasRx());
    ctx->Sub(r, a, b);
    check("Context::Sub(ct, ct)", same(bx_of(r), lanes(hb1, hb2, L, sub)) &&
                                      same(ax_of(r), lanes(ha1, ha2, L, sub)));
    ctx->Neg(r, a);
    check("Context::Neg", same(bx_of(r), lanes(hb1, none, L, neg)) &&
                              same(ax_of(r), lanes(ha1, none, L, neg)));
    {  // in place, res aliasing the second operand
      Ct c2;
      ctx->Copy(c2, b);
      ctx->Sub(c2, a, c2);
      check("Context::Sub in place", same(bx_of(c2), lanes(hb1, hb2, L, sub)) &&
                                         same(ax_of(c2), lanes(ha1, ha2, L, sub)));
    }
    // plaintext and constant operands
    std::vector<Complex> msg(1 << 10);
    for (auto &m : msg)
      m = Complex((next64() % 2001) / 1000.0 - 1.0,
                  (next64() % 2001) / 1000.0 - 1.0);
    Plaintext<word> pt;
    ctx->encoder_.Encode(pt, L - 1, 0x1p30, msg);
    const std::vector<word> hm = download(pt.mx_.data(), qw);
    Constant<word> cst;
    ctx->encoder_.EncodeConstant(cst, L - 1, 0x1p30, 0.75);
    const std::vector<word> hc = download(cst.cx_.data(), L);
    std::vector<word> hcb(qw);
    for (int l = 0; l < L; l++)
      for (size_t n = 0; n < kN; n++) hcb[l * kN + n] = hc[l];
    ctx->Add(r, a, pt);
    check("Context::Add(ct, pt)", same(bx_of(r), lanes(hb1, hm, L, add)) &&
                                      same(ax_of(r), ha1));
    ctx->Sub(r, pt, a);
    check("Context::Sub(pt, ct)", same(bx_of(r), lanes(hm, hb1, L, sub)) &&
                                      same(ax_of(r), lanes(ha1, none, L, neg)));
    ctx->Add(r, a, cst);
    check("Context::Add(ct, const)", same(bx_of(r), lanes(hb1, hcb, L, add)) &&
                                         same(ax_of(r), ha1));
    ctx->Sub(r, a, cst);
    check("Context::Sub(ct, const)", same(bx_of(r), lanes(hb1, hcb, L, sub)));
    ctx->Sub(r, cst, a);
    check("Context::Sub(const, ct)", same(bx_of(r), lanes(hcb, hb1, L, sub)) &&
                                         same(ax_of(r), lanes(ha1, none, L, neg)));
    ctx->Mult(r, a, pt);
    check("Context::Mult(ct, pt)", same(bx_of(r), lanes(hb1, hm, L, mul)) &&
                                       same(ax_of(r), lanes(ha1, hm, L, mul)) &&
                                       r.GetScale() == 0x1p60);
    ctx->Mult(r, a, cst);
    check("Context::Mult(ct, const)", same(bx_of(r), lanes(hb1, hcb, L, mul)) &&
                                          same(ax_of(r), lanes(ha1, hcb, L, mul)));
    {  // MultUnsafe at a lower level reads the operands' leading limbs
      const int lo = L - 4;
      ctx->MultUnsafe(r, a, pt, lo - 1);
      const std::vector<word> sb(hb1.begin(), hb1.begin() + lo * kN),
          sm(hm.begin(), hm.begin() + lo * kN);
      check("Context::MultUnsafe(ct, pt, level)",
            r.GetNP() == param.LevelToNP(lo - 1) &&
                same(bx_of(r), lanes(sb, sm, lo, mul)));
      Ct t;
      ctx->MultUnsafe(t, a, b, lo - 1);
      std::vector<word> tb(lo * kN), ta(lo * kN), tr(lo * kN);
      const std::vector<word> a1(hb1.begin(), hb1.begin() + lo * kN),
          a2(ha1.begin(), ha1.begin() + lo * kN),
          b1(hb2.begin(), hb2.begin() + lo * kN),
          b2(ha2.begin(), ha2.begin() + lo * kN);
      orc_tensor(tb.data(), ta.data(), tr.data(), a1.data(), a2.data(),
                 b1.data(), b2.data(), lo, main_p.data(), kLogN);
      check("Context::MultUnsafe(ct, ct, level)",
            t.HasRx() && same(bx_of(t), tb) && same(ax_of(t), ta) &&
                same(download(t.rx_.data(), lo * kN), tr));
    }
    // MadUnsafe: res += a * const, rx started from zero
    {
      Ct acc;
      ctx->Copy(acc, b);
      acc.SetScale(0x1p60);
      ctx->MadUnsafe(acc, a, cst);
      check("Context::MadUnsafe",
            same(bx_of(acc), lanes(hb2, lanes(hb1, hcb, L, mul), L, add)) &&
                same(ax_of(acc), lanes(ha2, lanes(ha1, hcb, L, mul), L, add)));
    }
    // MultImaginaryUnit: twice is Neg exactly; on an encoding, decode gives
    // i * m
    {
      Ct t, u;
      ctx->MultImaginaryUnit(t, a);
      ctx->MultImaginaryUnit(u, t);
      bool ok = same(bx_of(u), lanes(hb1, none, L, neg)) &&
                same(ax_of(u), lanes(ha1, none, L, neg));
      Ct e(np);
      upload(e.bx_.data(), hm);
      upload(e.ax_.data(), std::vector<word>(qw, 0));
      e.SetScale(0x1p30);
      e.SetNumSlots(1 << 10);
      ctx->MultImaginaryUnit(t, e);
      Plaintext<word> back(np);
      back.SetScale(0x1p30);
      back.SetNumSlots(1 << 10);
      upload(back.mx_.data(), bx_of(t));
      std::vector<Complex> dec;
      ctx->encoder_.Decode(dec, back);
      double err = 0;
      for (size_t i = 0; i < msg.size(); i++)
        err = std::max(err, std::abs(dec[i] - Complex(0, 1) * msg[i]));
      check("Context::MultImaginaryUnit (i*i = -1, decodes to i*m)",
            ok && err < 1e-3);
      // PermuteConjugate on the same encoding decodes to conj(m)
      ctx->PermuteConjugate(t, e);
      upload(back.mx_.data(), bx_of(t));
      ctx->encoder_.Decode(dec, back);
      err = 0;
      for (size_t i = 0; i < msg.size(); i++)
        err = std::max(err, std::abs(dec[i] - std::conj(msg[i])));
      check("Context::PermuteConjugate decodes to conj(m)", err < 1e-3);
    }
    // HConj / HConjAdd / HRotAdd against the oracle's MultKey + permutation
    {
      std::vector<word> mb(qw), ma(qw), pb(qw), pa(qw);
      orc_mult_key(mb.data(), ma.data(), hb1.data(), ha1.data(), kb.data(),
                   ka.data(), L, L, main_p.data(), aux_p.data(), alpha, kLogN);
      const uint32_t gconj = 2 * static_cast<uint32_t>(kN) - 1;
      orc_permute(pb.data(), mb.data(), L, kLogN, gconj);
      orc_permute(pa.data(), ma.data(), L, kLogN, gconj);
      ctx->HConj(r, a, key);
      check("Context::HConj", same(bx_of(r), pb) && same(ax_of(r), pa));
      ctx->HConjAdd(r, a, b, key);
      check("Context::HConjAdd", same(bx_of(r), lanes(pb, hb2, L, add)) &&
                                     same(ax_of(r), lanes(pa, ha2, L, add)));
      std::vector<word> hrb(qw), hra(qw);
      orc_hrot(hrb.data(), hra.data(), hb1.data(), ha1.data(), kb.data(),
               ka.data(), L, L, main_p.data(), aux_p.data(), alpha, kLogN, 5);
      Ct c2;
      ctx->Copy(c2, b);
      ctx->HRotAdd(c2, a, c2, key, 5);
      check("Context::HRotAdd (res aliases b)",
            same(bx_of(c2), lanes(hrb, hb2, L, add)) &&
                same(ax_of(c2), lanes(hra, ha2, L, add)));
    }
    // LevelDown by three levels: Mult by the level's unit constant, then
    // Rescale, per level (Context.cpp:917-929), and the encoding survives
    {
      const int top = L - 1, target = L - 4;
      std::vector<word> xb = hb1, xa = ha1;
      for (int lv = top; lv > target; lv--) {
        const int lim = lv + 1;
        Constant<word> c1;
        ctx->encoder_.EncodeConstant(c1, lv, param.GetScale(lv), 1.0);
        const std::vector<word> h1 = download(c1.cx_.data(), lim);
        std::vector<word> hb(lim * kN);
        for (int l = 0; l < lim; l++)
          for (size_t n = 0; n < kN; n++) hb[l * kN + n] = h1[l];
        std::vector<word> tb = lanes(xb, hb, lim, mul),
                          ta = lanes(xa, hb, lim, mul);
        xb.assign((lim - 1) * kN, 0);
        xa.assign((lim - 1) * kN, 0);
        orc_rescale(xb.data(), tb.data(), lim, main_p.data(), 1, kLogN);
        orc_rescale(xa.data(), ta.data(), lim, main_p.data(), 1, kLogN);
      }
      ctx->LevelDown(r, a, target);
      bool ok = r.GetNP() == param.LevelToNP(target) && same(bx_of(r), xb) &&
                same(ax_of(r), xa);
      Ct e(np), d;
      upload(e.bx_.data(), hm);
      upload(e.ax_.data(), std::vector<word>(qw, 0));
      e.SetScale(0x1p30);
      e.SetNumSlots(1 << 10);
      ctx->LevelDown(d, e, target);
      const NPInfo tnp = param.LevelToNP(target);
      Plaintext<word> back(tnp);
      back.SetScale(d.GetScale());
      back.SetNumSlots(1 << 10);
      upload(back.mx_.data(), bx_of(d));
      std::vector<Complex> dec;
      ctx->encoder_.Decode(dec, back);
      double err = 0;
      for (size_t i = 0; i < msg.size(); i++)
        err = std::max(err, std::abs(dec[i] - msg[i]));
      check("Context::LevelDown (oracle, and the encoding survives)",
            ok && err < 1e-3);
    }
  }
  // kernel ABI: the inverse NTT of 2 x 32 limbs out of place (the single
  // pass over residue classes) and in place (the two passes), plain and
  // centred, on the chain's 30- and 31-bit primes with arbitrary epilogue
  // constants, against the oracle's INTTAndMultConst (NTT.cu:743-813)
  {
    const ChainTables chain(kLogN, chain_k);
    const int nl = L + alpha, npoly = 2;
    const size_t w = static_cast<size_t>(nl) * kN;
    std::vector<word> x(npoly * w);
    for (int p = 0; p < npoly; p++) {
      const std::vector<word> v = uniform(chain_k, nl);
      std::copy(v.begin(), v.end(), x.begin() + p * w);
    }
    std::vector<word> cst(nl);
    for (int l = 0; l < nl; l++) cst[l] = next64() % chain_k[l];
    DevBuf dsrc(npoly * w * sizeof(word)), ddst(npoly * w * sizeof(word)),
        dcst(nl * sizeof(word));
    dcst.Upload(cst);
    chd_limb_map m{};
    m.num_q = nl;
    m.skip_lo = INT_MAX;
    for (int centre = 0; centre < 2; centre++) {
      std::vector<word> want(npoly * w);
      for (int p = 0; p < npoly; p++)
        for (int l = 0; l < nl; l++)
          orc_intt_mult_const(
              reinterpret_cast<int32_t *>(want.data() + p * w + l * kN),
              x.data() + p * w + l * kN, kLogN, chain_k[l], cst[l], centre);
      upload(dsrc.as<word>(), x);
      bool ok = chd_k_ntt_inv(&chain.tables(), &m, ddst.as<word>(),
                              static_cast<long long>(w), dsrc.as<word>(),
                              static_cast<long long>(w), nl, npoly,
                              dcst.as<word>(), centre, nullptr) == 0;
      ok = ok && same(download(ddst.as<word>(), npoly * w), want) &&
           same(download(dsrc.as<word>(), npoly * w), x);
      upload(ddst.as<word>(), x);
      ok = ok && chd_k_ntt_inv(&chain.tables(), &m, ddst.as<word>(),
                               static_cast<long long>(w), ddst.as<word>(),
                               static_cast<long long>(w), nl, npoly,
                               dcst.as<word>(), centre, nullptr) == 0;
      ok = ok && same(download(ddst.as<word>(), npoly * w), want);
      // the single pass over residue classes: the same words
      HipCheck(hipMemset(ddst.as<void>(), 0, npoly * w * sizeof(word)),
               "hipMemset");
      ok = ok && chd_k_ntt_inv_1p(&chain.tables(), &m, ddst.as<word>(),
                                  static_cast<long long>(w), dsrc.as<word>(),
                                  static_cast<long long>(w), nl, npoly,
                                  dcst.as<word>(), centre, nullptr) == 0;
      ok = ok && same(download(ddst.as<word>(), npoly * w), want);
      check(std::string("chd_k_ntt_inv 2 x 32 limbs, out of place, in place "
                        "and single pass") + (centre ? ", centred" : ""), ok);
    }
  }
  // an invalid call throws cheddar::Error instead of exiting
  {
    bool threw = false;
    try {
      Ct bad(param.LevelToNP(L - 2));
      Ct res;
      ctx->HMult(res, a, bad, key, true);
    } catch (const Error &) {
      threw = true;
    }
    check("NP mismatch throws cheddar::Error", threw);
  }
  std::printf("%s\n", g_fail == 0 ? "ALL PASS" : "FAILURES");
  return g_fail == 0 ? 0 : 1;
}
