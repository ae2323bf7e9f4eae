// Negacyclic NTT / INTT for N = 2^16 on gfx950.
//
// Four-step split N = 256 rows x 256 columns (index = row*256 + col).
// Forward Cooley-Tukey stages 0..7 pair rows (a column pass), stages 8..15
// pair columns inside one row (a row pass). Each pass is one kernel: one HBM
// read and one HBM write of every limb. Inside a pass a thread holds 16
// elements in registers, runs 4 radix-2 stages on them, exchanges through
// LDS, and runs the next 4 stages (radix-16 x radix-16).
//
// Semantics follow the reference exactly (bit-exact canonical outputs):
//   forward: y[i] = sum_j x_j psi^{(2 brev(i)+1) j}, twiddle psi_rev[m+i]
//            for butterfly group i of the stage with m groups
//            (include/core/NTTUtils.cuh:19-34, 62-87; src/core/NTT.cu:231-454)
//   inverse: Gentleman-Sande with psi_inv_rev[m+i], computes N*intt; the
//            N^-1 and any per-limb factor live in the epilogue constant,
//            applied as MontMul(x, c) (NTT.cu:23-229, 673-813).
// Butterfly arithmetic is the exact fp64 modular multiply of chd_device.h;
// values are kept unreduced in fp64 inside a pass (|x| < 2^40) and reduced to
// canonical u32 at each pass boundary.
#include "chd_device.h"
#include "kernel_common.h"
#include "ntt.h"

namespace chd {
namespace {

constexpr int kRows = 256;
constexpr int kCols = 256;
constexpr int kTileCols = 32;   // columns per column-pass workgroup
constexpr int kTileRows = 16;   // rows per row-pass workgroup
constexpr int kRowPad = kCols + kCols / 16;

struct Limb {
  int l;      // logical limb (dst index)
  int sl;     // src limb
  int ti;     // table index
  int ci;     // constant index
};

__device__ __forceinline__ Limb decode(const LimbMap &m, int j) {
  Limb r;
  r.l = j + (j >= m.skip_lo ? m.skip_len : 0);
  bool aux = r.l >= m.num_q;
  r.sl = r.l + (aux ? m.src_gap : 0);
  r.ti = m.tab_off + r.l + (aux ? m.tab_gap : 0);
  r.ci = r.l + (aux ? m.cst_gap : 0);
  return r;
}

__device__ __forceinline__ void ct_bfly(double &a, double &b, double w,
                                        double wq, double q) {
  double m = mulmod_f64(b, w, wq, q);
  b = a - m;
  a = a + m;
}

__device__ __forceinline__ void gs_bfly(double &a, double &b, double w,
                                        double wq, double q) {
  double d = a - b;
  a = a + b;
  b = mulmod_f64(d, w, wq, q);
}

// MontMul constant c (reference form) -> plain multiplier c * 2^-32 mod q
__device__ __forceinline__ double eff_const(uint32_t c, uint32_t rinv,
                                            double q, double qinv) {
  double r = static_cast<double>(rinv);
  double m = mulmod_f64(static_cast<double>(c), r, r * qinv, q);
  return static_cast<double>(reduce_f64(m, q, qinv));
}

__device__ __forceinline__ int pidx(int i) { return i + (i >> 4); }

// ------------------------------------------------------------------------
// forward, column pass: stages 0..7
// grid (kCols / kTileCols, limbs, polys), block 512
// ------------------------------------------------------------------------
template <bool kPre>
__global__ __launch_bounds__(512) void ntt_fwd_cols(NttArgs a) {
  __shared__ double xch[kRows * kTileCols];
  const Limb lb = decode(a.map, blockIdx.y);
  const uint32_t *src = a.src + blockIdx.z * a.src_pstride +
                        (static_cast<size_t>(lb.sl) << kLogN);
  uint32_t *dst =
      a.dst + blockIdx.z * a.dst_pstride + (static_cast<size_t>(lb.l) << kLogN);
  const double q = a.tab.qd[lb.ti];
  const double qinv = a.tab.qinvd[lb.ti];
  const double2 *tw =
      static_cast<const double2 *>(a.tab.tw_lo) + lb.ti * 256;
  const int c = threadIdx.x & (kTileCols - 1);
  const int rg = threadIdx.x / kTileCols;  // 0..15
  const int col = blockIdx.x * kTileCols + c;

  double x[16];
#pragma unroll
  for (int k = 0; k < 16; k++)
    x[k] = static_cast<double>(src[(rg + 16 * k) * kCols + col]);
  if constexpr (kPre) {
    double ce = eff_const(a.cst[lb.ci], a.tab.rinv[lb.ti], q, qinv);
    double ceq = ce * qinv;
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = mulmod_f64(x[k], ce, ceq, q);
  }
  // stages 0..3: rows rg + 16k, twiddles identical for every thread
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const int h = 8 >> s;
#pragma unroll
    for (int g = 0; g < (1 << s); g++) {
      const double2 w = tw[(1 << s) + g];
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++)
        ct_bfly(x[k], x[k + h], w.x, w.y, q);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; k++) xch[(rg + 16 * k) * kTileCols + c] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = xch[(16 * rg + k) * kTileCols + c];
  // stages 4..7: rows 16 rg + k
#pragma unroll
  for (int s = 4; s < 8; s++) {
    const int h = 8 >> (s - 4);
#pragma unroll
    for (int g = 0; g < (1 << (s - 4)); g++) {
      const double2 w = tw[(1 << s) + (rg << (s - 4)) + g];
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++)
        ct_bfly(x[k], x[k + h], w.x, w.y, q);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; k++)
    dst[(16 * rg + k) * kCols + col] = reduce_f64(x[k], q, qinv);
}

// ------------------------------------------------------------------------
// forward, row pass: stages 8..15 (in place on dst) + epilogue
// grid (kRows / kTileRows, limbs, polys), block 256
// ------------------------------------------------------------------------
template <int kEpi>
__global__ __launch_bounds__(256) void ntt_fwd_rows(NttArgs a) {
  __shared__ double xch[kTileRows * kRowPad];
  const Limb lb = decode(a.map, blockIdx.y);
  uint32_t *dst =
      a.dst + blockIdx.z * a.dst_pstride + (static_cast<size_t>(lb.l) << kLogN);
  const double q = a.tab.qd[lb.ti];
  const double qinv = a.tab.qinvd[lb.ti];
  const uint32_t *tw = a.tab.tw + (static_cast<size_t>(lb.ti) << kLogN);
  const int c = threadIdx.x & 15;
  const int r = threadIdx.x >> 4;
  const int row = blockIdx.x * kTileRows + r;
  uint32_t *base = dst + row * kCols;
  double *xr = xch + r * kRowPad;

  double x[16];
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = static_cast<double>(base[c + 16 * k]);
  // stages 8..11: columns c + 16k, twiddles depend on the row only
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const int h = 8 >> s;
#pragma unroll
    for (int g = 0; g < (1 << s); g++) {
      const double w = static_cast<double>(tw[(256 << s) + (row << s) + g]);
      const double wq = w * qinv;
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++)
        ct_bfly(x[k], x[k + h], w, wq, q);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; k++) xr[pidx(c + 16 * k)] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = xr[pidx(16 * c + k)];
  // stages 12..15: columns 16c + k
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const int h = 8 >> s;
#pragma unroll
    for (int g = 0; g < (1 << s); g++) {
      const double w = static_cast<double>(
          tw[(4096 << s) + (row << (4 + s)) + (c << s) + g]);
      const double wq = w * qinv;
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++)
        ct_bfly(x[k], x[k + h], w, wq, q);
    }
  }
  uint32_t out[16];
  if constexpr (kEpi == kEpiModDown) {
    const uint32_t rinv = a.tab.rinv[lb.ti];
    const double c2 = eff_const(a.cst2[lb.l], rinv, q, qinv);
    const double c2q = c2 * qinv;
    const int s2 = lb.l - a.src2_lo;
    const bool has2 = lb.l >= a.src2_lo && lb.l < a.src2_hi;
    if (has2) {
      const uint32_t *s2p = a.src2 + blockIdx.z * a.src2_pstride +
                            (static_cast<size_t>(s2) << kLogN) + row * kCols +
                            16 * c;
      double pe = 0.0, peq = 0.0;
      if (a.pad != nullptr) {
        pe = eff_const(a.pad[s2], rinv, q, qinv);
        peq = pe * qinv;
      }
#pragma unroll
      for (int k = 0; k < 16; k++) {
        double v = static_cast<double>(s2p[k]);
        if (a.pad != nullptr) v = mulmod_f64(v, pe, peq, q);
        out[k] = reduce_f64(mulmod_f64(v - x[k], c2, c2q, q), q, qinv);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 16; k++)
        out[k] = reduce_f64(mulmod_f64(-x[k], c2, c2q, q), q, qinv);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 16; k++) out[k] = reduce_f64(x[k], q, qinv);
  }
  uint4 *o4 = reinterpret_cast<uint4 *>(base + 16 * c);
#pragma unroll
  for (int v = 0; v < 4; v++)
    o4[v] = make_uint4(out[4 * v], out[4 * v + 1], out[4 * v + 2],
                       out[4 * v + 3]);
}

// ------------------------------------------------------------------------
// inverse, row pass: GS stages 15..8 (src -> dst)
// ------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ntt_inv_rows(NttArgs a) {
  __shared__ double xch[kTileRows * kRowPad];
  const Limb lb = decode(a.map, blockIdx.y);
  const uint32_t *src = a.src + blockIdx.z * a.src_pstride +
                        (static_cast<size_t>(lb.sl) << kLogN);
  uint32_t *dst =
      a.dst + blockIdx.z * a.dst_pstride + (static_cast<size_t>(lb.l) << kLogN);
  const double q = a.tab.qd[lb.ti];
  const double qinv = a.tab.qinvd[lb.ti];
  const uint32_t *tw = a.tab.itw + (static_cast<size_t>(lb.ti) << kLogN);
  const int c = threadIdx.x & 15;
  const int r = threadIdx.x >> 4;
  const int row = blockIdx.x * kTileRows + r;
  double *xr = xch + r * kRowPad;

  double x[16];
  const uint4 *i4 = reinterpret_cast<const uint4 *>(src + row * kCols + 16 * c);
#pragma unroll
  for (int v = 0; v < 4; v++) {
    uint4 u = i4[v];
    x[4 * v] = u.x;
    x[4 * v + 1] = u.y;
    x[4 * v + 2] = u.z;
    x[4 * v + 3] = u.w;
  }
  // stages 15..12: columns 16c + k
#pragma unroll
  for (int s = 3; s >= 0; s--) {
    const int h = 8 >> s;
#pragma unroll
    for (int g = 0; g < (1 << s); g++) {
      const double w = static_cast<double>(
          tw[(4096 << s) + (row << (4 + s)) + (c << s) + g]);
      const double wq = w * qinv;
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++)
        gs_bfly(x[k], x[k + h], w, wq, q);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; k++) xr[pidx(16 * c + k)] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = xr[pidx(c + 16 * k)];
  // stages 11..8: columns c + 16k
#pragma unroll
  for (int s = 3; s >= 0; s--) {
    const int h = 8 >> s;
#pragma unroll
    for (int g = 0; g < (1 << s); g++) {
      const double w = static_cast<double>(tw[(256 << s) + (row << s) + g]);
      const double wq = w * qinv;
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++)
        gs_bfly(x[k], x[k + h], w, wq, q);
    }
  }
  uint32_t *base = dst + row * kCols;
#pragma unroll
  for (int k = 0; k < 16; k++) base[c + 16 * k] = reduce_f64(x[k], q, qinv);
}

// ------------------------------------------------------------------------
// inverse, column pass: GS stages 7..0 (in place on dst) + constant epilogue
// ------------------------------------------------------------------------
template <int kEpi>
__global__ __launch_bounds__(512) void ntt_inv_cols(NttArgs a) {
  __shared__ double xch[kRows * kTileCols];
  const Limb lb = decode(a.map, blockIdx.y);
  uint32_t *dst =
      a.dst + blockIdx.z * a.dst_pstride + (static_cast<size_t>(lb.l) << kLogN);
  const double q = a.tab.qd[lb.ti];
  const double qinv = a.tab.qinvd[lb.ti];
  const double2 *tw =
      static_cast<const double2 *>(a.tab.itw_lo) + lb.ti * 256;
  const int c = threadIdx.x & (kTileCols - 1);
  const int rg = threadIdx.x / kTileCols;
  const int col = blockIdx.x * kTileCols + c;

  double x[16];
#pragma unroll
  for (int k = 0; k < 16; k++)
    x[k] = static_cast<double>(dst[(16 * rg + k) * kCols + col]);
#pragma unroll
  for (int s = 7; s >= 4; s--) {
    const int h = 8 >> (s - 4);
#pragma unroll
    for (int g = 0; g < (1 << (s - 4)); g++) {
      const double2 w = tw[(1 << s) + (rg << (s - 4)) + g];
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++)
        gs_bfly(x[k], x[k + h], w.x, w.y, q);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; k++) xch[(16 * rg + k) * kTileCols + c] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = xch[(rg + 16 * k) * kTileCols + c];
#pragma unroll
  for (int s = 3; s >= 0; s--) {
    const int h = 8 >> s;
#pragma unroll
    for (int g = 0; g < (1 << s); g++) {
      const double2 w = tw[(1 << s) + g];
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++)
        gs_bfly(x[k], x[k + h], w.x, w.y, q);
    }
  }
  const double ce = eff_const(a.cst[lb.ci], a.tab.rinv[lb.ti], q, qinv);
  const double ceq = ce * qinv;
#pragma unroll
  for (int k = 0; k < 16; k++) {
    double v = mulmod_f64(x[k], ce, ceq, q);
    uint32_t o;
    if constexpr (kEpi == kEpiConstCentre)
      o = static_cast<uint32_t>(centre_f64(v, q, qinv));
    else
      o = reduce_f64(v, q, qinv);
    dst[(rg + 16 * k) * kCols + col] = o;
  }
}

}  // namespace

hipError_t launch_ntt_fwd(const NttArgs &a, int num_limbs, int num_polys,
                          bool pre_const, int epilogue, hipStream_t s) {
  if (num_limbs <= 0 || num_polys <= 0) return hipSuccess;
  dim3 gc(kCols / kTileCols, num_limbs, num_polys);
  dim3 gr(kRows / kTileRows, num_limbs, num_polys);
  if (pre_const)
    hipLaunchKernelGGL(ntt_fwd_cols<true>, gc, dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL(ntt_fwd_cols<false>, gc, dim3(512), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (epilogue == kEpiModDown)
    hipLaunchKernelGGL(ntt_fwd_rows<kEpiModDown>, gr, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(ntt_fwd_rows<kEpiStore>, gr, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_ntt_inv(const NttArgs &a, int num_limbs, int num_polys,
                          int epilogue, hipStream_t s) {
  if (num_limbs <= 0 || num_polys <= 0) return hipSuccess;
  dim3 gr(kRows / kTileRows, num_limbs, num_polys);
  dim3 gc(kCols / kTileCols, num_limbs, num_polys);
  hipLaunchKernelGGL(ntt_inv_rows, gr, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // the column pass works in place on dst
  NttArgs b = a;
  b.map.src_gap = 0;
  if (epilogue == kEpiConstCentre)
    hipLaunchKernelGGL(ntt_inv_cols<kEpiConstCentre>, gc, dim3(512), 0, s, b);
  else
    hipLaunchKernelGGL(ntt_inv_cols<kEpiConst>, gc, dim3(512), 0, s, b);
  return hipGetLastError();
}

}  // namespace chd

using namespace chd;

extern "C" int chd_k_ntt_fwd(const chd_tables *t, const chd_limb_map *m,
                             uint32_t *dst, long long dst_pstride,
                             const uint32_t *src, long long src_pstride,
                             int num_limbs, int num_polys,
                             const uint32_t *pre_cst, void *stream) {
  if (!t || !m || !dst || !src || num_limbs < 0 || num_polys < 0)
    return set_error(CHD_ERR_ARG, "chd_k_ntt_fwd: invalid argument");
  NttArgs a{};
  a.src = src;
  a.dst = dst;
  a.src_pstride = src_pstride;
  a.dst_pstride = dst_pstride;
  a.map = *m;
  a.tab = *t;
  a.cst = pre_cst;
  hipError_t e = launch_ntt_fwd(a, num_limbs, num_polys, pre_cst != nullptr,
                                kEpiStore, static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return set_error(CHD_ERR_HIP, std::string("chd_k_ntt_fwd: ") +
                                      hipGetErrorString(e));
  return 0;
}

extern "C" int chd_k_ntt_fwd_moddown(const chd_tables *t,
                                     const chd_limb_map *m, uint32_t *dst,
                                     int num_limbs, const uint32_t *src2,
                                     int src2_lo, int src2_hi,
                                     const uint32_t *inv_prod,
                                     const uint32_t *pad, void *stream) {
  if (!t || !m || !dst || !inv_prod || num_limbs < 0 ||
      (src2 == nullptr && src2_hi > src2_lo) || src2 == dst)
    return set_error(CHD_ERR_ARG, "chd_k_ntt_fwd_moddown: invalid argument");
  NttArgs a{};
  a.src = dst;
  a.dst = dst;
  a.map = *m;
  a.map.src_gap = 0;
  a.tab = *t;
  a.src2 = src2;
  a.src2_lo = src2_lo;
  a.src2_hi = src2_hi;
  a.cst2 = inv_prod;
  a.pad = pad;
  hipError_t e = launch_ntt_fwd(a, num_limbs, 1, false, kEpiModDown,
                                static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return set_error(CHD_ERR_HIP, std::string("chd_k_ntt_fwd_moddown: ") +
                                      hipGetErrorString(e));
  return 0;
}

extern "C" int chd_k_ntt_inv(const chd_tables *t, const chd_limb_map *m,
                             uint32_t *dst, long long dst_pstride,
                             const uint32_t *src, long long src_pstride,
                             int num_limbs, int num_polys, const uint32_t *cst,
                             int centre, void *stream) {
  if (!t || !m || !dst || !src || !cst || num_limbs < 0 || num_polys < 0)
    return set_error(CHD_ERR_ARG, "chd_k_ntt_inv: invalid argument");
  NttArgs a{};
  a.src = src;
  a.dst = dst;
  a.src_pstride = src_pstride;
  a.dst_pstride = dst_pstride;
  a.map = *m;
  a.tab = *t;
  a.cst = cst;
  hipError_t e =
      launch_ntt_inv(a, num_limbs, num_polys,
                     centre ? kEpiConstCentre : kEpiConst,
                     static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return set_error(CHD_ERR_HIP, std::string("chd_k_ntt_inv: ") +
                                      hipGetErrorString(e));
  return 0;
}
