// BConv: the base-conversion matrix product of ModUp / ModDown / Rescale
// (reference kernel ModSwitchMatrixMult, src/core/ModSwitch.cu:23-171).
//
//   dst[pos(k)][n] = sum_i c_i[n] * T[k][i] * 2^-32  mod p_k
//
// c_i are centred int32 residues (the INTT epilogue's output) and T is the
// reference's "double Montgomery" table centre(qhat_i R^2 mod p_k). The
// kernel folds the 2^-32 into the table once on the host:
// U[k][i] = centre(T[k][i] * 2^-32 mod p_k), split U = Uhi * 2^16 + Ulo with
// Ulo in [0, 2^16). Then sum_i c_i Uhi and sum_i c_i Ulo are exact fp64
// FMA chains (|c| < 2^30: partial sums below 2^50 for up to 16 sources), the
// high part is reduced mod p, recombined as rhi * 2^16 + slo (exact) and
// reduced to [0, p). All FMAs run at full fp64 VALU rate on gfx950.
//
// Layout: one thread per coefficient n, all sources held in registers; the
// table is wave-uniform (scalar loads). grid (N / 256, dst chunks).
#include <algorithm>
#include <cstring>
#include <vector>

#include "chd_device.h"
#include "cheddar_kernels.h"
#include "kernel_common.h"

namespace chd {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxSrc = 16;
constexpr int kDstChunk = 12;

struct BconvTab {   // per (k, i): {Uhi, Ulo} as doubles
  double hi, lo;
};

struct BconvBatch {
  chd_bconv_job job[CHD_MAX_JOBS];
};

template <int kSrc>
__global__ __launch_bounds__(kThreads) void bconv_kernel(chd_tables t,
                                                         chd_limb_map m,
                                                         BconvBatch b) {
  const chd_bconv_job &jb = b.job[blockIdx.z];
  const int n = blockIdx.x * kThreads + threadIdx.x;
  const int k0 = blockIdx.y * kDstChunk;
  const int k1 = min(jb.dst_len, k0 + kDstChunk);
  if (k0 >= k1) return;
  const int ns = kSrc > 0 ? kSrc : jb.src_len;
  const int32_t *__restrict__ src = jb.src;
  const BconvTab *__restrict__ tab = static_cast<const BconvTab *>(jb.table);
  double c[kMaxSrc];
#pragma unroll
  for (int i = 0; i < kMaxSrc; i++)
    if (i < ns) c[i] = static_cast<double>(src[(static_cast<size_t>(i) << kLogN) + n]);
  for (int k = k0; k < k1; k++) {
    const int pos = k + (k >= jb.skip_lo ? jb.skip_len : 0);
    const bool aux = pos >= m.num_q;
    const int ti = m.tab_off + pos + (aux ? m.tab_gap : 0);
    const double p = t.qd[ti];
    const double pinv = t.qinvd[ti];
    const BconvTab *row = tab + static_cast<size_t>(k) * ns;
    double shi = 0.0, slo = 0.0;
#pragma unroll
    for (int i = 0; i < kMaxSrc; i++) {
      if (i < ns) {
        const BconvTab e = row[i];
        shi = __builtin_fma(c[i], e.hi, shi);
        slo = __builtin_fma(c[i], e.lo, slo);
      }
    }
    const double rhi = __builtin_fma(-__builtin_rint(shi * pinv), p, shi);
    const double v = __builtin_fma(rhi, 65536.0, slo);
    jb.dst[(static_cast<size_t>(pos) << kLogN) + n] = reduce_f64(v, p, pinv);
  }
}

}  // namespace
}  // namespace chd

using namespace chd;

extern "C" long long chd_bconv_table_size(int src_len, int dst_len) {
  if (src_len < 1 || dst_len < 1) return 0;
  return static_cast<long long>(src_len) * dst_len * sizeof(BconvTab);
}

extern "C" int chd_bconv_table_pack(void *host_out, const int32_t *table_ref,
                                    const uint32_t *dst_primes, int src_len,
                                    int dst_len) {
  if (!host_out || !table_ref || !dst_primes || src_len < 1 ||
      src_len > kMaxSrc || dst_len < 1)
    return set_error(CHD_ERR_ARG, "chd_bconv_table_pack: invalid argument");
  BconvTab *out = static_cast<BconvTab *>(host_out);
  for (int k = 0; k < dst_len; k++) {
    const uint64_t p = dst_primes[k];
    // 2^-32 mod p by Fermat-free extended Euclid on (2^32 mod p, p)
    int64_t r0 = static_cast<int64_t>(p), r1 = static_cast<int64_t>((1ull << 32) % p);
    int64_t t0 = 0, t1 = 1;
    while (r1 != 0) {
      int64_t qq = r0 / r1, tmp = t0 - qq * t1;
      t0 = t1;
      t1 = tmp;
      tmp = r0 - qq * r1;
      r0 = r1;
      r1 = tmp;
    }
    const uint64_t rinv = static_cast<uint64_t>(t0 < 0 ? t0 + static_cast<int64_t>(p) : t0);
    for (int i = 0; i < src_len; i++) {
      int64_t tv = table_ref[static_cast<size_t>(k) * src_len + i];
      uint64_t tu = static_cast<uint64_t>(tv < 0 ? tv + static_cast<int64_t>(p) : tv);
      uint64_t u = tu * rinv % p;
      int64_t uc = static_cast<int64_t>(u);
      if (u > (p >> 1)) uc -= static_cast<int64_t>(p);
      int64_t lo = uc & 0xFFFF;
      int64_t hi = (uc - lo) / 65536;
      out[static_cast<size_t>(k) * src_len + i] =
          BconvTab{static_cast<double>(hi), static_cast<double>(lo)};
    }
  }
  return 0;
}

extern "C" int chd_k_bconv_batch(const chd_tables *t, const chd_limb_map *m,
                                 const chd_bconv_job *jobs, int num_jobs,
                                 void *stream) {
  if (!t || !m || !jobs || num_jobs < 1 || num_jobs > CHD_MAX_JOBS)
    return set_error(CHD_ERR_ARG, "chd_k_bconv_batch: invalid argument");
  BconvBatch b{};
  int max_dst = 0, src_len = jobs[0].src_len;
  bool same_src = true;
  for (int j = 0; j < num_jobs; j++) {
    const chd_bconv_job &jb = jobs[j];
    if (!jb.dst || !jb.src || !jb.table || jb.src_len < 1 ||
        jb.src_len > kMaxSrc || jb.dst_len < 1 || jb.skip_len < 0)
      return set_error(CHD_ERR_ARG, "chd_k_bconv_batch: invalid job");
    b.job[j] = jb;
    max_dst = std::max(max_dst, jb.dst_len);
    same_src = same_src && jb.src_len == src_len;
  }
  dim3 g(kN / kThreads, (max_dst + kDstChunk - 1) / kDstChunk, num_jobs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int sl = same_src ? src_len : 0;
  switch (sl) {
    case 1:
      hipLaunchKernelGGL(bconv_kernel<1>, g, dim3(kThreads), 0, s, *t, *m, b);
      break;
    case 8:
      hipLaunchKernelGGL(bconv_kernel<8>, g, dim3(kThreads), 0, s, *t, *m, b);
      break;
    case 9:
      hipLaunchKernelGGL(bconv_kernel<9>, g, dim3(kThreads), 0, s, *t, *m, b);
      break;
    default:
      hipLaunchKernelGGL(bconv_kernel<0>, g, dim3(kThreads), 0, s, *t, *m, b);
      break;
  }
  return check_launch("chd_k_bconv_batch");
}

extern "C" int chd_k_bconv(const chd_tables *t, const chd_limb_map *m,
                           uint32_t *dst, const int32_t *src, int src_len,
                           int dst_len, const void *table, void *stream) {
  if (!t || !m || !dst || !src || !table || src_len < 1 ||
      src_len > kMaxSrc || dst_len < 1)
    return set_error(CHD_ERR_ARG, "chd_k_bconv: invalid argument");
  chd_bconv_job j{dst, src, table, src_len, dst_len, m->skip_lo, m->skip_len};
  return chd_k_bconv_batch(t, m, &j, 1, stream);
}
