// CKKS encoder (src/core/Encode.cpp). Each step cites the reference lines
// whose operation order it keeps; the arithmetic is IEEE double with no
// contraction (this file is compiled with -ffp-contract=off), so complex
// products are (ac - bd, ad + bc) with each product rounded, as the
// reference's host build (-O3, no FMA target) computes them.
#include <cmath>
#include <cstring>

#include "cheddar.h"
#include "prime_math.h"

namespace cheddar {

namespace {

int Log2CeilInt(int a) {
  AssertTrue(a > 0, "Log2Ceil: only positive values");
  int r = 0;
  while ((1 << r) < a) r++;
  return r;
}

// CommonUtils.h:162-178: in-place bit-reversal permutation
void BitReverseVector(std::vector<Complex> &data) {
  const int n = static_cast<int>(data.size());
  const int bits = Log2CeilInt(n);
  for (int i = 0; i < n; i++) {
    const int j = static_cast<int>(pm::bitrev(static_cast<uint32_t>(i), bits));
    if (i < j) std::swap(data[i], data[j]);
  }
}

uint32_t Pow2Mod(int e, uint32_t p) {  // 2^e mod p, e >= 0
  uint64_t r = 1 % p, b = 2 % p;
  for (; e > 0; e >>= 1) {
    if (e & 1) r = r * b % p;
    b = b * b % p;
  }
  return static_cast<uint32_t>(r);
}

// BigInt(double) then BigInt::Mod: the double truncated toward zero
// (mp_set_double / mpz_set_d, BigInt_tommath.cpp:22-26, BigInt_gmp.cpp:22-25)
// and reduced to [0, p) (mp_mod / mpz_mod take the divisor's sign).
uint32_t TruncMod(double x, uint32_t p) {
  AssertTrue(std::isfinite(x), "Encode: message value is not finite");
  const double t = std::trunc(x);
  // |t| < p (almost every coefficient of an encoded message): no division
  if (t >= 0.0 && t < static_cast<double>(p)) return static_cast<uint32_t>(t);
  if (t < 0.0 && -t < static_cast<double>(p))
    return p - static_cast<uint32_t>(-t);
  if (std::fabs(t) < 0x1p63) {
    int64_t r = static_cast<int64_t>(t) % static_cast<int64_t>(p);
    if (r < 0) r += p;
    return static_cast<uint32_t>(r);
  }
  // |t| >= 2^63 is the integer mant * 2^(e - 53) with a 53-bit mantissa
  int e = 0;
  const double fr = std::frexp(std::fabs(t), &e);
  const uint64_t mant = static_cast<uint64_t>(std::ldexp(fr, 53));
  uint64_t r = (mant % p) * Pow2Mod(e - 53, p) % p;
  if (t < 0 && r != 0) r = p - r;
  return static_cast<uint32_t>(r);
}

// Multi-word unsigned integers, little-endian 32-bit words, for the CRT of
// Decode (the reference's BigInt products and sums, Encode.cpp:210-236).
using Words = std::vector<uint32_t>;

Words MulSmall(const Words &a, uint32_t b) {
  Words r(a.size() + 1, 0);
  uint64_t carry = 0;
  for (size_t i = 0; i < a.size(); i++) {
    const uint64_t t = static_cast<uint64_t>(a[i]) * b + carry;
    r[i] = static_cast<uint32_t>(t);
    carry = t >> 32;
  }
  r[a.size()] = static_cast<uint32_t>(carry);
  while (r.size() > 1 && r.back() == 0) r.pop_back();
  return r;
}

// a >= b, both n words
bool GreaterEq(const uint32_t *a, const uint32_t *b, size_t n) {
  for (size_t i = n; i-- > 0;)
    if (a[i] != b[i]) return a[i] > b[i];
  return true;
}

// a -= b, both n words, a >= b
void SubInPlace(uint32_t *a, const uint32_t *b, size_t n) {
  uint64_t borrow = 0;
  for (size_t i = 0; i < n; i++) {
    const uint64_t t = static_cast<uint64_t>(a[i]) - b[i] - borrow;
    a[i] = static_cast<uint32_t>(t);
    borrow = (t >> 63) & 1;
  }
}

// libtommath's mp_get_double (the reference's default BigInt backend,
// BigInt_tommath.cpp:49, USE_GMP off in CMakeLists.txt:34): the magnitude's
// 60-bit digits from the most significant, d = d * 2^60 + (double)digit,
// each step rounded to nearest; then the sign.
double TommathGetDouble(const uint32_t *mag, size_t n, bool negative) {
  size_t bits = n * 32;
  while (bits > 0 && ((mag[(bits - 1) / 32] >> ((bits - 1) % 32)) & 1) == 0)
    bits--;
  const size_t used = (bits + 59) / 60;
  double d = 0.0;
  for (size_t k = used; k-- > 0;) {
    uint64_t digit = 0;
    for (int b = 0; b < 60; b++) {
      const size_t bit = k * 60 + b;
      if (bit >= n * 32) break;
      digit |= static_cast<uint64_t>((mag[bit / 32] >> (bit % 32)) & 1) << b;
    }
    d = d * 0x1p60 + static_cast<double>(digit);
  }
  return negative ? -d : d;
}

}  // namespace

// Encode.cpp:10-21: twiddle i = e^(2 pi sqrt(-1) i / M), M = 2N
Encoder<uint32_t>::Encoder(const Parameter<word> &param,
                           const NTTHandler<word> &ntt_handler)
    : Encoder(param) {
  ntt_handler_ = &ntt_handler;
}

Encoder<uint32_t>::Encoder(const Parameter<word> &param)
    : param_(param), ntt_handler_(nullptr), m_(2 * param.degree_), twiddle_(m_) {
  for (int i = 0; i < m_; i++)
    twiddle_[i] = std::polar(1.0, 2.0 * M_PI * i / m_);
}

// Encode.cpp:84-109
void Encoder<uint32_t>::SpecialIFFT(std::vector<Complex> &data) const {
  const int slots = static_cast<int>(data.size());
  AssertTrue(slots == (1 << Log2CeilInt(slots)), "Power of 2 num slots only");
  for (int stride = slots / 2; stride >= 1; stride /= 2) {
    const int st8 = stride << 3;
    const int gap = m_ / st8;
    for (int i = 0; i < slots; i += 2 * stride) {
      for (int j = 0; j < stride; j++) {
        const int tw = (st8 - (param_.GetGaloisFactor(j) % st8)) * gap;
        const Complex x = data[i + j] + data[i + j + stride];
        Complex y = data[i + j] - data[i + j + stride];
        y *= twiddle_[tw];
        data[i + j] = x;
        data[i + j + stride] = y;
      }
    }
  }
  BitReverseVector(data);
  for (int i = 0; i < slots; i++) data[i] /= slots;
}

// Encode.cpp:111-133
void Encoder<uint32_t>::SpecialFFT(std::vector<Complex> &data) const {
  const int slots = static_cast<int>(data.size());
  AssertTrue(slots == (1 << Log2CeilInt(slots)), "Power of 2 num slots only");
  BitReverseVector(data);
  for (int stride = 1; stride < slots; stride *= 2) {
    const int st8 = stride << 3;
    const int gap = m_ / st8;
    for (int i = 0; i < slots; i += 2 * stride) {
      for (int j = 0; j < stride; j++) {
        const int tw = (param_.GetGaloisFactor(j) % st8) * gap;
        const Complex x = data[i + j];
        Complex y = data[i + j + stride];
        y *= twiddle_[tw];
        data[i + j] = x + y;
        data[i + j + stride] = x - y;
      }
    }
  }
}

// Encode.cpp:135-190 (ComplexVectorToPlaintext) after the SpecialIFFT of
// EncodeWorker (Encode.cpp:34-43)
std::vector<uint32_t> Encoder<uint32_t>::CoefficientResidues(
    int level, double scale, std::vector<Complex> data, int num_aux) const {
  SpecialIFFT(data);
  const int slots = static_cast<int>(data.size());
  const int n = param_.degree_;
  const int half = n / 2;
  AssertTrue(slots <= half, "ComplexVectorToPlaintext: Too many slots");
  const int gap = half / slots;
  const NPInfo np = param_.LevelToNP(level, num_aux);
  const std::vector<word> primes = param_.GetPrimeVector(np);
  std::vector<word> mx(primes.size() * static_cast<size_t>(n), 0);
  for (int i = 0; i < slots; i++) {
    const Complex v = data[i] * scale;
    const double re = v.real(), im = v.imag();
    for (size_t j = 0; j < primes.size(); j++) {
      mx[j * n + static_cast<size_t>(i) * gap] = TruncMod(re, primes[j]);
      mx[j * n + static_cast<size_t>(i) * gap + half] = TruncMod(im, primes[j]);
    }
  }
  return mx;
}

// Encode.cpp:23-43: pad to a power of two, residues, NTT(mc = true)
void Encoder<uint32_t>::Encode(Plaintext<word> &ptxt, int level, double scale,
                               const std::vector<Complex> &message,
                               int num_aux) const {
  AssertTrue(ntt_handler_ != nullptr, "Encode: host-only encoder");
  std::vector<Complex> padded = PadToPowerOfTwo(message);
  const int slots = static_cast<int>(padded.size());
  const std::vector<word> mx =
      CoefficientResidues(level, scale, std::move(padded), num_aux);
  EncodeResidues(ptxt, level, scale, slots, mx, num_aux);
}

std::vector<Complex> Encoder<uint32_t>::PadToPowerOfTwo(
    const std::vector<Complex> &message) {
  const int len = static_cast<int>(message.size());
  std::vector<Complex> padded(static_cast<size_t>(1) << Log2CeilInt(len));
  std::copy(message.begin(), message.end(), padded.begin());
  return padded;
}

// the device half of Encode: upload the residues, NTT with Montgomery
// conversion
void Encoder<uint32_t>::EncodeResidues(Plaintext<word> &ptxt, int level,
                                       double scale, int slots,
                                       const std::vector<word> &mx,
                                       int num_aux) const {
  AssertTrue(ntt_handler_ != nullptr, "Encode: host-only encoder");
  const NPInfo np = param_.LevelToNP(level, num_aux);
  AssertTrue(mx.size() == static_cast<size_t>(np.GetNumTotal()) *
                              static_cast<size_t>(param_.degree_),
             "Encode: residues do not match the level");
  Plaintext<word> out(np, param_.degree_);
  HipCheck(hipMemcpyAsync(out.mx_.data(), mx.data(), mx.size() * sizeof(word),
                          hipMemcpyHostToDevice, CurrentStream()),
           "hipMemcpyAsync");
  // the aux limbs follow the q limbs directly: views with their aux size
  const int aux_words = num_aux * param_.degree_;
  DvView<word> v = out.mx_.View(aux_words);
  ntt_handler_->NTT(v, np, out.mx_.ConstView(aux_words), true);
  // mx is the caller's host memory: the copy has to finish before it goes
  HipCheck(hipStreamSynchronize(CurrentStream()), "hipStreamSynchronize");
  out.SetNumSlots(slots);
  out.SetScale(scale);
  ptxt = std::move(out);
}

// Encode.cpp:248-273
void Encoder<uint32_t>::EncodeConstant(Constant<word> &constant, int level,
                                       double scale, double number,
                                       int num_aux) const {
  AssertTrue(ntt_handler_ != nullptr, "EncodeConstant: host-only encoder");
  const double v = number * scale;
  const NPInfo np = param_.LevelToNP(level, num_aux);
  const std::vector<word> primes = param_.GetPrimeVector(np);
  std::vector<word> cx(primes.size());
  for (size_t i = 0; i < primes.size(); i++)
    cx[i] = pm::to_mont(TruncMod(v, primes[i]), primes[i]);
  Constant<word> out(np);
  HipCheck(hipMemcpyAsync(out.cx_.data(), cx.data(), cx.size() * sizeof(word),
                          hipMemcpyHostToDevice, CurrentStream()),
           "hipMemcpyAsync");
  HipCheck(hipStreamSynchronize(CurrentStream()), "hipStreamSynchronize");
  out.SetScale(scale);
  constant = std::move(out);
}

// Encode.cpp:45-82 and 192-246 (PlaintextToComplexVector)
void Encoder<uint32_t>::Decode(std::vector<Complex> &message,
                               const Plaintext<word> &ptxt) const {
  AssertTrue(ntt_handler_ != nullptr, "Decode: host-only encoder");
  const NPInfo np = ptxt.GetNP();
  AssertTrue(np.num_aux_ == 0, "Decode: Aux primes not supported");
  const std::vector<word> primes = param_.GetPrimeVector(np);
  const int lp = static_cast<int>(primes.size());
  const int n = param_.degree_;
  const int half = n / 2;
  const int slots = ptxt.GetNumSlots();
  AssertTrue(slots == (1 << Log2CeilInt(slots)),
             "ComplexVectorToPlaintext: Power of 2 num slots only");
  AssertTrue(slots <= half, "PlaintextToComplexVector: Too many slots");
  const int gap = half / slots;

  // iCRT constants (N prod_{k != i} q_k)^-1 mod q_i, not in Montgomery form
  std::vector<word> icrt(lp);
  for (int i = 0; i < lp; i++) {
    uint32_t prod = 1;
    for (int j = 0; j < lp; j++)
      if (j != i) prod = pm::mulmod(prod, primes[j] % primes[i], primes[i]);
    prod = pm::mulmod(prod, static_cast<uint32_t>(n) % primes[i], primes[i]);
    icrt[i] = pm::invmod(prod, primes[i]);
  }
  DeviceVector<word> icrt_dv(lp);
  Plaintext<word> tmp(np, n);
  std::vector<word> res(static_cast<size_t>(lp) * n);
  HipCheck(hipMemcpyAsync(icrt_dv.data(), icrt.data(), lp * sizeof(word),
                          hipMemcpyHostToDevice, CurrentStream()),
           "hipMemcpyAsync");
  DvView<word> tv = tmp.mx_.View();
  ntt_handler_->INTTAndMultConst(tv, np, ptxt.mx_.ConstView(),
                                icrt_dv.ConstView());
  HipCheck(hipMemcpyAsync(res.data(), tmp.mx_.data(), res.size() * sizeof(word),
                          hipMemcpyDeviceToHost, CurrentStream()),
           "hipMemcpyAsync");
  HipCheck(hipStreamSynchronize(CurrentStream()), "hipStreamSynchronize");

  // Q, Q / q_j and floor(Q / 2)
  Words q{1};
  for (int j = 0; j < lp; j++) q = MulSmall(q, primes[j]);
  std::vector<Words> qhat(lp);
  for (int j = 0; j < lp; j++) {
    Words w{1};
    for (int k = 0; k < lp; k++)
      if (k != j) w = MulSmall(w, primes[k]);
    qhat[j] = w;
  }
  const size_t width = q.size() + 1;  // sum < lp * Q < 2^32 * Q
  q.resize(width, 0);
  Words half_q(width, 0);
  for (size_t i = 0; i < width; i++)
    half_q[i] = (q[i] >> 1) | (i + 1 < width ? q[i + 1] << 31 : 0);
  for (auto &w : qhat) w.resize(width, 0);
  Words acc(width), mag(width);

  // sum_j r_j (Q / q_j) mod Q, centred into (-Q/2, Q/2], then to double
  auto value = [&](size_t idx) {
    std::fill(acc.begin(), acc.end(), 0u);
    for (int j = 0; j < lp; j++) {
      const uint64_t r = res[static_cast<size_t>(j) * n + idx];
      uint64_t carry = 0;
      for (size_t w = 0; w < width; w++) {
        const uint64_t t = acc[w] + r * qhat[j][w] + carry;
        acc[w] = static_cast<uint32_t>(t);
        carry = t >> 32;
      }
    }
    while (GreaterEq(acc.data(), q.data(), width))
      SubInPlace(acc.data(), q.data(), width);
    if (GreaterEq(half_q.data(), acc.data(), width))
      return TommathGetDouble(acc.data(), width, false);
    mag = q;  // acc > Q/2: the value is acc - Q
    SubInPlace(mag.data(), acc.data(), width);
    return TommathGetDouble(mag.data(), width, true);
  };

  const double scale = ptxt.GetScale();
  message.assign(slots, Complex());
  for (int i = 0; i < slots; i++) {
    const double re = value(static_cast<size_t>(i) * gap) / scale;
    const double im = value(static_cast<size_t>(i) * gap + half) / scale;
    message[i] = Complex(re, im);
  }
  SpecialFFT(message);
}

}  // namespace cheddar
