#include "device_tables.h"

#include "prime_math.h"

namespace cheddar {

void HipCheck(hipError_t e, const char *what) {
  if (e != hipSuccess)
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void DevBuf::Resize(size_t bytes) {
  if (bytes == bytes_) return;
  Release();
  if (bytes == 0) return;
  HipCheck(hipMalloc(&ptr_, bytes), "hipMalloc");
  bytes_ = bytes;
}

void DevBuf::Upload(const void *host, size_t bytes) {
  if (bytes > bytes_) throw std::runtime_error("DevBuf::Upload: overflow");
  HipCheck(hipMemcpy(ptr_, host, bytes, hipMemcpyHostToDevice), "hipMemcpy");
}

void DevBuf::Release() {
  if (ptr_ != nullptr) (void)hipFree(ptr_);
  ptr_ = nullptr;
  bytes_ = 0;
}

// twiddle tables as in NTTHandler::PopulateTwiddleFactors (NTT.cu:1233-1299)
ChainTables::ChainTables(int log_degree, const std::vector<uint32_t> &primes)
    : primes_(primes) {
  if (log_degree != 16)
    throw std::invalid_argument("only log_degree 16 is supported");
  const int n = 1 << log_degree;
  const size_t T = primes.size();
  std::vector<int32_t> qinv(T);
  std::vector<uint32_t> ninv(T), ninv_mont(T), r2(T);
  std::vector<uint32_t> tw(T * n), itw(T * n);
  // the single-pass inverse's twists: psi^-(s e_k), e_k = 2 brev(k) + 1
  // over log N - 2 bits, for the residue classes s = 0..3 of its output
  // (class 0's row is ToMont(1): every class runs the same code)
  const int m4 = n / 4;
  std::vector<uint32_t> twist(T * 4 * m4);
  std::vector<uint32_t> ipow(2 * n);
  for (size_t i = 0; i < T; i++) {
    const uint32_t q = primes[i];
    if (q >= (1u << 31) || q % (2u * n) != 1)
      throw std::invalid_argument("prime " + std::to_string(q) +
                                  " is not an NTT-friendly prime below 2^31");
    qinv[i] = pm::inv_mod_base(q);
    ninv[i] = pm::invmod(static_cast<uint32_t>(n % q), q);
    ninv_mont[i] = pm::to_mont(ninv[i], q);
    r2[i] = pm::to_mont(pm::to_mont(1, q), q);
    const uint32_t psi = pm::primitive_root(2u * n, q);
    const uint32_t psi_inv = pm::invmod(psi, q);
    uint64_t p = 1, pi = 1;
    uint32_t *t = tw.data() + i * n;
    uint32_t *it = itw.data() + i * n;
    for (int j = 0; j < n; j++) {
      const uint32_t r = pm::bitrev(static_cast<uint32_t>(j), log_degree);
      t[r] = pm::to_mont(static_cast<uint32_t>(p), q);
      it[r] = pm::to_mont(static_cast<uint32_t>(pi), q);
      p = p * psi % q;
      pi = pi * psi_inv % q;
    }
    // psi^-e for e < 2N (psi has order 2N)
    uint64_t e1 = 1;
    for (int e = 0; e < 2 * n; e++) {
      ipow[e] = static_cast<uint32_t>(e1);
      e1 = e1 * psi_inv % q;
    }
    for (int s = 0; s < 4; s++)
      for (int k = 0; k < m4; k++) {
        const uint32_t ek =
            2u * pm::bitrev(static_cast<uint32_t>(k), log_degree - 2) + 1u;
        twist[(i * 4 + s) * m4 + k] =
            pm::to_mont(ipow[(s * ek) % (2u * n)], q);
      }
  }
  q_.Upload(primes);
  qinv_.Upload(qinv);
  tw_.Upload(tw);
  itw_.Upload(itw);
  twist_.Upload(twist);
  ninv_.Upload(ninv);
  ninv_mont_.Upload(ninv_mont);
  r2_.Upload(r2);
  tab_.q = q_.as<uint32_t>();
  tab_.qinv = qinv_.as<int32_t>();
  tab_.tw = tw_.as<uint32_t>();
  tab_.itw = itw_.as<uint32_t>();
  tab_.twist = twist_.as<uint32_t>();
}

}  // namespace cheddar
