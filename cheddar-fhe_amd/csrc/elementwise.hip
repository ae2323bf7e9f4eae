// Element-wise kernels of the key-switch path (HBM-bound): Tensor,
// CPAccum/CPAccumAdd (the evaluation-key inner product), Permute.
//
// One thread owns 4 consecutive coefficients of one limb (128-bit loads and
// stores); grid (N / 1024, limbs). Arithmetic is the reference's signed
// Montgomery product MontMul(a, b) = a b 2^-32 mod q, canonical outputs.
#include "chd_device.h"
#include "cheddar_kernels.h"
#include "kernel_common.h"

namespace chd {
namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 4;
constexpr int kCoefPerBlock = kThreads * kPerThread;

struct LimbIdx {
  int l;
  bool aux;
  uint32_t q;
  int32_t qinv;
};

__device__ __forceinline__ LimbIdx limb_of(const chd_tables &t,
                                           const chd_limb_map &m) {
  LimbIdx r;
  r.l = blockIdx.y + (static_cast<int>(blockIdx.y) >= m.skip_lo ? m.skip_len : 0);
  r.aux = r.l >= m.num_q;
  int ti = m.tab_off + r.l + (r.aux ? m.tab_gap : 0);
  r.q = t.q[ti];
  r.qinv = t.qinv[ti];
  return r;
}

__device__ __forceinline__ uint4 ld4(const uint32_t *p) {
  return *reinterpret_cast<const uint4 *>(p);
}
// streaming read of data used once (the giant steps' plaintexts): the hint
// keeps it from evicting the baby steps the other waves still read
__device__ __forceinline__ uint4 ld4_once(const uint32_t *p) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st4(uint32_t *p, uint4 v) {
  *reinterpret_cast<uint4 *>(p) = v;
}
__device__ __forceinline__ uint32_t get(const uint4 &v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Tensor (ElementWise.cu:504-546)
__global__ __launch_bounds__(kThreads) void tensor_kernel(
    chd_tables t, chd_limb_map m, uint32_t *bx, uint32_t *ax, uint32_t *rx,
    const uint32_t *b1, const uint32_t *a1, const uint32_t *b2,
    const uint32_t *a2) {
  LimbIdx li = limb_of(t, m);
  size_t o = (static_cast<size_t>(li.l) << kLogN) +
             blockIdx.x * kCoefPerBlock + threadIdx.x * kPerThread;
  size_t si = o + (li.aux ? static_cast<size_t>(m.src_gap) << kLogN : 0);
  uint4 vb1 = ld4(b1 + si), va1 = ld4(a1 + si);
  uint4 vb2 = ld4(b2 + si), va2 = ld4(a2 + si);
  uint32_t ob[4], oa[4], orr[4];
  const int32_t q = static_cast<int32_t>(li.q);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int32_t x1 = get(vb1, i), y1 = get(va1, i);
    int32_t x2 = get(vb2, i), y2 = get(va2, i);
    int32_t s1 = (x1 - q) + y1;  // [-q, q-2]
    int32_t s2 = (x2 - q) + y2;
    uint32_t mid = mont_mul(s1, s2, li.q, li.qinv);
    uint32_t bb = mont_mul(x1, x2, li.q, li.qinv);
    uint32_t aa = mont_mul(y1, y2, li.q, li.qinv);
    mid = sub_mod(mid, bb, li.q);
    mid = sub_mod(mid, aa, li.q);
    ob[i] = bb;
    oa[i] = mid;
    orr[i] = aa;
  }
  st4(bx + o, make_uint4(ob[0], ob[1], ob[2], ob[3]));
  st4(ax + o, make_uint4(oa[0], oa[1], oa[2], oa[3]));
  st4(rx + o, make_uint4(orr[0], orr[1], orr[2], orr[3]));
}

// TensorSquare (ElementWise.cu:549-575)
__global__ __launch_bounds__(kThreads) void tensor_square_kernel(
    chd_tables t, chd_limb_map m, uint32_t *bx, uint32_t *ax, uint32_t *rx,
    const uint32_t *b1, const uint32_t *a1) {
  LimbIdx li = limb_of(t, m);
  size_t o = (static_cast<size_t>(li.l) << kLogN) +
             blockIdx.x * kCoefPerBlock + threadIdx.x * kPerThread;
  size_t si = o + (li.aux ? static_cast<size_t>(m.src_gap) << kLogN : 0);
  uint4 vb = ld4(b1 + si), va = ld4(a1 + si);
  uint32_t ob[4], oa[4], orr[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int32_t x = get(vb, i), y = get(va, i);
    ob[i] = mont_mul(x, x, li.q, li.qinv);
    uint32_t xy = mont_mul(x, y, li.q, li.qinv);
    oa[i] = add_mod(xy, xy, li.q);
    orr[i] = mont_mul(y, y, li.q, li.qinv);
  }
  st4(bx + o, make_uint4(ob[0], ob[1], ob[2], ob[3]));
  st4(ax + o, make_uint4(oa[0], oa[1], oa[2], oa[3]));
  st4(rx + o, make_uint4(orr[0], orr[1], orr[2], orr[3]));
}

struct AccumArgs {
  uint32_t *dst[CHD_MAX_POLY];
  const uint32_t *src0[CHD_MAX_POLY];
  long long src0_gap;
  chd_accum_src s[CHD_MAX_ACCUM];
};

// CPAccum / CPAccumAdd (ElementWise.cu:225-366)
template <int kPoly, bool kConst, bool kHasSrc0>
__global__ __launch_bounds__(kThreads) void cpaccum_kernel(chd_tables t,
                                                           chd_limb_map m,
                                                           AccumArgs a,
                                                           int num_accum) {
  LimbIdx li = limb_of(t, m);
  const int c0 = blockIdx.x * kCoefPerBlock + threadIdx.x * kPerThread;
  const size_t o = (static_cast<size_t>(li.l) << kLogN) + c0;
  uint32_t acc[kPoly][4];
#pragma unroll
  for (int p = 0; p < kPoly; p++) {
    if constexpr (kHasSrc0) {
      uint4 v = ld4(a.src0[p] + o + (li.aux ? a.src0_gap : 0));
      acc[p][0] = v.x;
      acc[p][1] = v.y;
      acc[p][2] = v.z;
      acc[p][3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) acc[p][i] = 0;
    }
  }
  for (int j = 0; j < num_accum; j++) {
    const chd_accum_src &s = a.s[j];
    const size_t so = o + (li.aux ? s.src_gap : 0);
    uint32_t cm[4];
    if constexpr (kConst) {
      uint32_t cv = s.common[li.l + (li.aux ? s.common_gap : 0)];
#pragma unroll
      for (int i = 0; i < 4; i++) cm[i] = cv;
    } else {
      uint4 cv = ld4(s.common + o + (li.aux ? s.common_gap : 0));
      cm[0] = cv.x;
      cm[1] = cv.y;
      cm[2] = cv.z;
      cm[3] = cv.w;
    }
#pragma unroll
    for (int p = 0; p < kPoly; p++) {
      uint4 v = ld4(s.src[p] + so);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        uint32_t mm = mont_mul(static_cast<int32_t>(cm[i]),
                               static_cast<int32_t>(get(v, i)), li.q, li.qinv);
        acc[p][i] = add_mod(acc[p][i], mm, li.q);
      }
    }
  }
#pragma unroll
  for (int p = 0; p < kPoly; p++)
    st4(a.dst[p] + o, make_uint4(acc[p][0], acc[p][1], acc[p][2], acc[p][3]));
}

struct PermArgs {
  uint32_t *dst[CHD_MAX_POLY];
  const uint32_t *src[CHD_MAX_POLY];
};

// Permute (ElementWise.cu:370-391)
template <int kPoly>
__global__ __launch_bounds__(kThreads) void permute_kernel(chd_limb_map m,
                                                           PermArgs a,
                                                           uint32_t galois) {
  const int l = blockIdx.y;
  const bool aux = l >= m.num_q;
  const size_t base = static_cast<size_t>(l) << kLogN;
  const size_t sbase = base + (aux ? static_cast<size_t>(m.src_gap) << kLogN : 0);
  const int c0 = blockIdx.x * kCoefPerBlock + threadIdx.x * kPerThread;
  uint32_t idx[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    uint32_t x = c0 + i;
    uint32_t e = (__brev(x) >> (32 - (kLogN + 1))) + 1;
    idx[i] = __brev(e * galois - 1) >> (32 - (kLogN + 1));
  }
#pragma unroll
  for (int p = 0; p < kPoly; p++) {
    const uint32_t *s = a.src[p] + sbase;
    st4(a.dst[p] + base + c0,
        make_uint4(s[idx[0]], s[idx[1]], s[idx[2]], s[idx[3]]));
  }
}

// galois index map of Permute (ElementWise.cu:370-391): dst[x] = src[perm(x)]
__device__ __forceinline__ uint32_t perm_index(uint32_t x, uint32_t galois) {
  const uint32_t e = (__brev(x) >> (32 - (kLogN + 1))) + 1;
  return __brev(e * galois - 1) >> (32 - (kLogN + 1));
}

__global__ __launch_bounds__(kThreads) void zero_kernel(uint4 *dst,
                                                      long long n4) {
  const long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n4) dst[i] = make_uint4(0, 0, 0, 0);
}

struct PermAccArgs {
  uint32_t *dst[CHD_MAX_POLY];
  const uint32_t *src0[CHD_MAX_POLY];
  long long src0_gap;
  chd_perm_src s[CHD_MAX_ACCUM];
};

// PermuteAccum / PermuteAccumAdd (ElementWise.cu:395-501)
template <int kPoly>
__global__ __launch_bounds__(kThreads) void permute_accum_kernel(
    chd_tables t, chd_limb_map m, PermAccArgs a, int num_src) {
  const LimbIdx li = limb_of(t, m);
  const size_t base = static_cast<size_t>(li.l) << kLogN;
  const int c0 = blockIdx.x * kCoefPerBlock + threadIdx.x * kPerThread;
  uint32_t acc[kPoly][4];
#pragma unroll
  for (int p = 0; p < kPoly; p++) {
    if (a.src0[0] != nullptr) {
      const uint4 v = ld4(a.src0[p] + base + c0 + (li.aux ? a.src0_gap : 0));
      acc[p][0] = v.x;
      acc[p][1] = v.y;
      acc[p][2] = v.z;
      acc[p][3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) acc[p][i] = 0;
    }
  }
  for (int j = 0; j < num_src; j++) {
    const chd_perm_src &s = a.s[j];
    uint32_t idx[4];
#pragma unroll
    for (int i = 0; i < 4; i++) idx[i] = perm_index(c0 + i, s.galois);
    const size_t sb = base + (li.aux ? s.src_gap : 0);
#pragma unroll
    for (int p = 0; p < kPoly; p++) {
      const uint32_t *sp = s.src[p] + sb;
#pragma unroll
      for (int i = 0; i < 4; i++) acc[p][i] = add_mod(acc[p][i], sp[idx[i]], li.q);
    }
  }
#pragma unroll
  for (int p = 0; p < kPoly; p++)
    st4(a.dst[p] + base + c0, make_uint4(acc[p][0], acc[p][1], acc[p][2], acc[p][3]));
}

// Hoisted baby step (BSFusedKernel, src/extension/Hoist.cu:20-78): the ModUp
// of a is read once per coefficient and reused by every rotation; the
// automorphism is applied as a scatter with the inverse galois factor, so the
// key loads stay coalesced.
__global__ __launch_bounds__(kThreads) void bs_fused_kernel(chd_tables t,
                                                          chd_limb_map m,
                                                          chd_bs_args a) {
  const LimbIdx li = limb_of(t, m);
  const size_t loff = static_cast<size_t>(li.l) << kLogN;
  const int c0 = blockIdx.x * kCoefPerBlock + threadIdx.x * kPerThread;
  uint32_t u[CHD_MAX_BS_GROUPS][4];
  for (int g = 0; g < a.beta; g++) {
    const int own_lo = group_lo(g, a.alpha, a.group_shift);
    const int own_hi = group_hi(g, a.alpha, a.group_shift, a.num_q);
    const uint32_t *src = (li.l >= own_lo && li.l < own_hi)
                              ? a.d + loff
                              : a.modup + g * a.group_stride + loff;
    const uint4 v = ld4(src + c0);
    u[g][0] = v.x;
    u[g][1] = v.y;
    u[g][2] = v.z;
    u[g][3] = v.w;
  }
  uint32_t pb[4] = {0, 0, 0, 0};
  if (!li.aux) {
    // PseudoModUp of b (ModSwitch.cu:414-428): MontMul(b, p_prod)
    const int32_t pp = static_cast<int32_t>(a.p_prod[li.l]);
    const uint4 v = ld4(a.ct_b + loff + c0);
    pb[0] = mont_mul(static_cast<int32_t>(v.x), pp, li.q, li.qinv);
    pb[1] = mont_mul(static_cast<int32_t>(v.y), pp, li.q, li.qinv);
    pb[2] = mont_mul(static_cast<int32_t>(v.z), pp, li.q, li.qinv);
    pb[3] = mont_mul(static_cast<int32_t>(v.w), pp, li.q, li.qinv);
  }
  const size_t koff = loff + (li.aux ? a.key_gap : 0);
  const uint32_t qn = 0u - static_cast<uint32_t>(li.qinv);
  for (int k = 0; k < a.num_rot; k++) {
    uint32_t tb[4], ta[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      tb[i] = pb[i];
      ta[i] = 0;
    }
    // key products of canonical residues summed in 64 bits, four at most
    // per Montgomery reduction (the same residue as summing MontMuls);
    // the key tiles are read once, with the streaming hint
    uint64_t sb[4] = {0, 0, 0, 0}, sa[4] = {0, 0, 0, 0};
    for (int g = 0; g < a.beta; g++) {
      const uint4 kb = ld4_once(a.kb[k][g] + koff + c0);
      const uint4 ka = ld4_once(a.ka[k][g] + koff + c0);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint64_t uv = u[g][i];
        sb[i] += uv * get(kb, i);
        sa[i] += uv * get(ka, i);
      }
      if ((g & 3) == 3 || g == a.beta - 1) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          tb[i] = add_mod(tb[i], reduce_sum4(sb[i], li.q, qn), li.q);
          ta[i] = add_mod(ta[i], reduce_sum4(sa[i], li.q, qn), li.q);
          sb[i] = sa[i] = 0;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t di = perm_index(c0 + i, a.galois[k]);
      a.dst_b[k][loff + di] = tb[i];
      a.dst_a[k][loff + di] = ta[i];
    }
  }
}

// Hoisted giant step (GSFusedKernel, src/extension/Hoist.cu:80-118): a
// thread owns 4 coefficients of one limb and the accumulators of every giant
// step of the launch; each baby step is loaded once and multiplied into all
// of them (baby steps outer, giant steps inner).
__global__ __launch_bounds__(kThreads) void gs_fused_kernel(chd_tables t,
                                                          chd_limb_map m,
                                                          chd_gs_args a) {
  const LimbIdx li = limb_of(t, m);
  const size_t o = (static_cast<size_t>(li.l) << kLogN) +
                   blockIdx.x * kCoefPerBlock + threadIdx.x * kPerThread;
  uint32_t rb[CHD_GS_MAX_GS][4], ra[CHD_GS_MAX_GS][4];
#pragma unroll
  for (int g = 0; g < CHD_GS_MAX_GS; g++) {
    if (g < a.num_gs && a.add_to_dst) {
      const uint4 vb = ld4(a.dst_b[g] + o), va = ld4(a.dst_a[g] + o);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        rb[g][i] = get(vb, i);
        ra[g][i] = get(va, i);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) rb[g][i] = ra[g][i] = 0;
    }
  }
  for (int b = 0; b < a.num_bs; b++) {
    const uint4 xb = ld4(a.bs_b[b] + o), xa = ld4(a.bs_a[b] + o);
#pragma unroll
    for (int g = 0; g < CHD_GS_MAX_GS; g++) {
      if (g < a.num_gs && a.pt[g][b] != nullptr) {
        const uint4 mv = ld4(a.pt[g][b] + o);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int32_t mm = static_cast<int32_t>(get(mv, i));
          rb[g][i] = add_mod(rb[g][i],
                             mont_mul(mm, static_cast<int32_t>(get(xb, i)),
                                      li.q, li.qinv), li.q);
          ra[g][i] = add_mod(ra[g][i],
                             mont_mul(mm, static_cast<int32_t>(get(xa, i)),
                                      li.q, li.qinv), li.q);
        }
      }
    }
  }
#pragma unroll
  for (int g = 0; g < CHD_GS_MAX_GS; g++) {
    if (g < a.num_gs) {
      st4(a.dst_b[g] + o, make_uint4(rb[g][0], rb[g][1], rb[g][2], rb[g][3]));
      st4(a.dst_a[g] + o, make_uint4(ra[g][0], ra[g][1], ra[g][2], ra[g][3]));
    }
  }
}


// Wide giant-step accumulation: the 4 waves of a workgroup share 256
// coefficients of one limb (4 per lane, 16-byte loads) and each owns kGw of
// the launch's 4 kGw giant steps, so a launch reads every baby step once
// from HBM for all of them (the other waves' reads of it hit in cache).
// Plaintext addresses come from a device table (wave-uniform scalar loads);
// every entry is valid (absent pairs point at a zero plaintext) and baby
// steps come in fours (padded with zero ones), so the loop has no branches.
// Four products of a giant step are summed in 64 bits and reduced once,
// which equals the sum of their MontMuls mod q (the reference's
// MontMul-then-add, GSFusedKernel of Hoist.cu:80-118, in canonical form).
// kSmall (q < 2^30): a sum of four products of canonical residues is below
// 4 q^2 < q 2^32, so one Montgomery reduction maps it to (sum) 2^-32 in
// [0, 2q), and the accumulators stay in [0, 2q) until the final store.
// Otherwise (q < 2^31) the sum is reduced by reduce_sum4 to [0, q) and
// accumulated canonically.
template <int kGw, bool kSmall, bool kTiled>
__device__ __forceinline__ void gs_wide_body(const chd_gs_wide_args &a,
                                             const LimbIdx &li) {
  const uint32_t q = li.q;
  const uint32_t qn = 0u - static_cast<uint32_t>(li.qinv);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const size_t o = (static_cast<size_t>(li.l) << kLogN) +
                   blockIdx.x * (64 * kPerThread) + (threadIdx.x & 63) * kPerThread;
  const int g0 = wave * kGw;
  // tiled plaintexts (chd_k_gs_pack_tiled): this workgroup's block of this
  // limb, every (giant, baby) pair 256 words apart, lane part included
  [[maybe_unused]] const int tiled_rows = a.tiled_rows;
  [[maybe_unused]] const uint32_t *tile =
      kTiled ? a.pt_tiled +
                   ((static_cast<size_t>(li.l) * (kN / (64 * kPerThread)) +
                     blockIdx.x) *
                        static_cast<size_t>(tiled_rows) * a.pt_stride
                    << 8) +
                   (threadIdx.x & 63) * kPerThread
             : nullptr;
  uint32_t rb[kGw][4], ra[kGw][4];
#pragma unroll
  for (int g = 0; g < kGw; g++) {
    if (a.add_to_dst) {
      const uint4 vb = ld4(a.dst_b[g0 + g] + o), va = ld4(a.dst_a[g0 + g] + o);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        rb[g][i] = get(vb, i);
        ra[g][i] = get(va, i);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) rb[g][i] = ra[g][i] = 0u;
    }
  }
  auto acc = [&](uint32_t &r, uint64_t t) {
    if constexpr (kSmall) {
      const uint32_t m = static_cast<uint32_t>(t) * qn;
      const uint32_t d =
          static_cast<uint32_t>((static_cast<uint64_t>(m) * q + t) >> 32);
      const uint32_t s = r + d;  // [0, 4q)
      r = s < s - 2 * q ? s : s - 2 * q;
    } else {
      r = add_mod(r, reduce_sum4(t, q, qn), q);
    }
  };
  for (int b0 = 0; b0 < a.num_bs; b0 += 4) {
    uint4 xb[4], xa[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      xb[j] = ld4(a.bs_b[b0 + j] + o);
      xa[j] = ld4(a.bs_a[b0 + j] + o);
    }
    const uint32_t *const *row = a.pt_table + g0 * a.pt_stride + b0;
#pragma unroll
    for (int g = 0; g < kGw; g++) {
      uint4 mv[4];
      if constexpr (kTiled) {
        // giant steps past tiled_rows (padding) are not computed
        if (g0 + g >= tiled_rows) continue;
        // this pair's 256 coefficients of the block; the next baby step
        // 256 words on
        const uint32_t *p =
            tile + (static_cast<size_t>((g0 + g) * a.pt_stride + b0) << 8);
#pragma unroll
        for (int j = 0; j < 4; j++) mv[j] = ld4_once(p + (j << 8));
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++)
          mv[j] = ld4_once(row[g * a.pt_stride + j] + o);
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        uint64_t tb = 0, ta = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint64_t mm = get(mv[j], i);
          tb += mm * get(xb[j], i);
          ta += mm * get(xa[j], i);
        }
        acc(rb[g][i], tb);
        acc(ra[g][i], ta);
      }
    }
  }
#pragma unroll
  for (int g = 0; g < kGw; g++) {
    if constexpr (kTiled)
      if (g0 + g >= tiled_rows) break;
    if constexpr (kSmall) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        rb[g][i] = rb[g][i] < rb[g][i] - q ? rb[g][i] : rb[g][i] - q;
        ra[g][i] = ra[g][i] < ra[g][i] - q ? ra[g][i] : ra[g][i] - q;
      }
    }
    st4(a.dst_b[g0 + g] + o, make_uint4(rb[g][0], rb[g][1], rb[g][2], rb[g][3]));
    st4(a.dst_a[g0 + g] + o, make_uint4(ra[g][0], ra[g][1], ra[g][2], ra[g][3]));
  }
}

template <int kGw, bool kTiled>
__global__ __launch_bounds__(kThreads) void gs_wide_kernel(chd_tables t,
                                                         chd_limb_map m,
                                                         chd_gs_wide_args a) {
  const LimbIdx li = limb_of(t, m);
  if (li.q < (1u << 30))
    gs_wide_body<kGw, true, kTiled>(a, li);
  else
    gs_wide_body<kGw, false, kTiled>(a, li);
}

// Tiled plaintext copy for gs_wide_kernel: grid (N / 256 blocks, limbs,
// rows); the 4 waves of a workgroup copy the row's pt_stride baby steps of
// one 256-coefficient block, 1 KiB per wave instruction.
__global__ __launch_bounds__(kThreads) void gs_pack_tiled_kernel(
    const uint32_t *const *pt_table, int rows, int pt_stride,
    uint32_t *dst) {
  const int k = blockIdx.x, l = blockIdx.y, g = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const size_t so = (static_cast<size_t>(l) << kLogN) + (k << 8) + lane * 4;
  uint32_t *d = dst +
                ((((static_cast<size_t>(l) * (kN >> 8) + k) * rows + g) *
                  pt_stride)
                 << 8) +
                lane * 4;
  for (int b = wave; b < pt_stride; b += kThreads / 64)
    st4(d + (static_cast<size_t>(b) << 8),
        ld4_once(pt_table[g * pt_stride + b] + so));
}

// One row back out of the tiled copy: grid (N / 256 blocks, dst limbs), the
// row's pt_stride baby steps of one block, 1 KiB per wave instruction.
__global__ __launch_bounds__(kThreads) void gs_untile_row_kernel(
    const uint32_t *tiled, int rows, int pt_stride, int g, int dst_limbs,
    uint32_t *dst) {
  const int k = blockIdx.x, l = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t *s = tiled +
                      ((((static_cast<size_t>(l) * (kN >> 8) + k) * rows + g) *
                        pt_stride)
                       << 8) +
                      lane * 4;
  uint32_t *d = dst + (static_cast<size_t>(l) << kLogN) + (k << 8) + lane * 4;
  for (int b = wave; b < pt_stride; b += kThreads / 64)
    st4(d + (static_cast<size_t>(b) * dst_limbs << kLogN),
        ld4_once(s + (static_cast<size_t>(b) << 8)));
}

// Element-wise arithmetic (ElementWise.cu:33-220 Sum / Sub / Neg / Mult /
// AddConst / SubConst / SubOppositeConst / MultConst, 600-660
// MultImaginaryUnit; Basic.cuh:169-260 for the canonical forms).
__device__ __forceinline__ uint32_t ew_neg(uint32_t a, uint32_t q) {
  return a == 0 ? 0u : q - a;
}

__global__ __launch_bounds__(kThreads) void elementwise_kernel(chd_tables t,
                                                             chd_limb_map m,
                                                             chd_ew_args a) {
  const LimbIdx li = limb_of(t, m);
  const size_t loff = static_cast<size_t>(li.l) << kLogN;
  const int c0 = blockIdx.x * kCoefPerBlock + threadIdx.x * kPerThread;
  const size_t aoff = loff + (li.aux ? static_cast<size_t>(a.a_gap) << kLogN : 0);
  const size_t boff = loff + (li.aux ? static_cast<size_t>(a.b_gap) << kLogN : 0);
  const uint32_t q = li.q;
  const int32_t qi = li.qinv;
  uint32_t cv = 0;
  const int op = a.op;
  if (op >= CHD_EW_ADD_CONST && op <= CHD_EW_MULT_CONST)
    cv = a.cst[li.l + (li.aux ? a.cst_gap : 0)];
  if (op == CHD_EW_MULT_I) {
    const int ti = m.tab_off + li.l + (li.aux ? m.tab_gap : 0);
    cv = t.tw[(static_cast<size_t>(ti) << kLogN) + 1];  // ToMont(psi^(N/2))
    if (c0 >= kN / 2) cv = ew_neg(cv, q);
  }
  for (int p = 0; p < a.num_poly; p++) {
    const uint4 x = ld4(a.a[p] + aoff + c0);
    uint4 y = make_uint4(0, 0, 0, 0);
    if (op == CHD_EW_ADD || op == CHD_EW_SUB || op == CHD_EW_MULT)
      y = ld4(a.b[p] + boff + c0);
    else if (op == CHD_EW_PMULT)
      y = ld4(a.b[0] + boff + c0);
    uint32_t xv[4] = {x.x, x.y, x.z, x.w};
    const uint32_t yv[4] = {y.x, y.y, y.z, y.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      switch (op) {
        case CHD_EW_ADD: o[i] = add_mod(xv[i], yv[i], q); break;
        case CHD_EW_SUB: o[i] = sub_mod(xv[i], yv[i], q); break;
        case CHD_EW_NEG: o[i] = ew_neg(xv[i], q); break;
        case CHD_EW_MULT:
        case CHD_EW_PMULT:
          o[i] = mont_mul(static_cast<int32_t>(xv[i]),
                          static_cast<int32_t>(yv[i]), q, qi);
          break;
        case CHD_EW_ADD_CONST: o[i] = add_mod(xv[i], cv, q); break;
        case CHD_EW_SUB_CONST: o[i] = sub_mod(xv[i], cv, q); break;
        case CHD_EW_SUB_OPP_CONST: o[i] = sub_mod(cv, xv[i], q); break;
        case CHD_EW_MULT_CONST:
        case CHD_EW_MULT_I:
          o[i] = mont_mul(static_cast<int32_t>(xv[i]),
                          static_cast<int32_t>(cv), q, qi);
          break;
        default: o[i] = xv[i]; break;
      }
    }
    st4(a.dst[p] + loff + c0, make_uint4(o[0], o[1], o[2], o[3]));
  }
}
}  // namespace
}  // namespace chd

using namespace chd;

extern "C" int chd_k_tensor(const chd_tables *t, const chd_limb_map *m,
                            uint32_t *bx, uint32_t *ax, uint32_t *rx,
                            const uint32_t *b1, const uint32_t *a1,
                            const uint32_t *b2, const uint32_t *a2,
                            int num_limbs, void *stream) {
  if (!t || !m || !bx || !ax || !rx || !b1 || !a1 || !b2 || !a2 ||
      num_limbs < 0)
    return set_error(CHD_ERR_ARG, "chd_k_tensor: invalid argument");
  if (num_limbs == 0) return 0;
  dim3 g(kN / kCoefPerBlock, num_limbs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (b1 == b2 && a1 == a2)
    hipLaunchKernelGGL(tensor_square_kernel, g, dim3(kThreads), 0, s, *t, *m,
                       bx, ax, rx, b1, a1);
  else
    hipLaunchKernelGGL(tensor_kernel, g, dim3(kThreads), 0, s, *t, *m, bx, ax,
                       rx, b1, a1, b2, a2);
  return check_launch("chd_k_tensor");
}

extern "C" int chd_k_cpaccum(const chd_tables *t, const chd_limb_map *m,
                             uint32_t *const *dst, int num_polys,
                             const uint32_t *const *src0, long long src0_gap,
                             const chd_accum_src *srcs, int num_accum,
                             int const_accum, int num_limbs, void *stream) {
  if (!t || !m || !dst || !srcs || num_polys < 1 ||
      num_polys > CHD_MAX_POLY || num_accum < 1 || num_accum > CHD_MAX_ACCUM ||
      num_limbs < 0)
    return set_error(CHD_ERR_ARG, "chd_k_cpaccum: invalid argument");
  if (num_limbs == 0) return 0;
  AccumArgs a{};
  for (int p = 0; p < num_polys; p++) {
    a.dst[p] = dst[p];
    a.src0[p] = src0 ? src0[p] : nullptr;
  }
  a.src0_gap = src0_gap;
  for (int j = 0; j < num_accum; j++) a.s[j] = srcs[j];
  dim3 g(kN / kCoefPerBlock, num_limbs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  bool has0 = src0 != nullptr;
#define CHD_ACCUM_LAUNCH(P, C, S0)                                          \
  hipLaunchKernelGGL((cpaccum_kernel<P, C, S0>), g, dim3(kThreads), 0, s, \
                     *t, *m, a, num_accum)
#define CHD_ACCUM_POLY(P)                         \
  if (const_accum) {                              \
    if (has0) CHD_ACCUM_LAUNCH(P, true, true);    \
    else CHD_ACCUM_LAUNCH(P, true, false);        \
  } else {                                        \
    if (has0) CHD_ACCUM_LAUNCH(P, false, true);   \
    else CHD_ACCUM_LAUNCH(P, false, false);       \
  }
  if (num_polys == 1) {
    CHD_ACCUM_POLY(1)
  } else if (num_polys == 2) {
    CHD_ACCUM_POLY(2)
  } else {
    CHD_ACCUM_POLY(3)
  }
#undef CHD_ACCUM_POLY
#undef CHD_ACCUM_LAUNCH
  return check_launch("chd_k_cpaccum");
}

extern "C" int chd_k_permute(const chd_limb_map *m, uint32_t *const *dst,
                             const uint32_t *const *src, int num_polys,
                             int num_limbs, uint32_t galois, void *stream) {
  if (!m || !dst || !src || num_polys < 1 || num_polys > CHD_MAX_POLY ||
      num_limbs < 0 || (galois & 1u) == 0)
    return set_error(CHD_ERR_ARG, "chd_k_permute: invalid argument");
  if (num_limbs == 0) return 0;
  PermArgs a{};
  for (int p = 0; p < num_polys; p++) {
    if (dst[p] == src[p])
      return set_error(CHD_ERR_ARG, "chd_k_permute: in-place not supported");
    a.dst[p] = dst[p];
    a.src[p] = src[p];
  }
  dim3 g(kN / kCoefPerBlock, num_limbs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (num_polys == 1)
    hipLaunchKernelGGL(permute_kernel<1>, g, dim3(kThreads), 0, s, *m, a,
                       galois);
  else if (num_polys == 2)
    hipLaunchKernelGGL(permute_kernel<2>, g, dim3(kThreads), 0, s, *m, a,
                       galois);
  else
    hipLaunchKernelGGL(permute_kernel<3>, g, dim3(kThreads), 0, s, *m, a,
                       galois);
  return check_launch("chd_k_permute");
}

extern "C" int chd_k_permute_accum(const chd_tables *t, const chd_limb_map *m,
                                   uint32_t *const *dst, int num_polys,
                                   const uint32_t *const *src0,
                                   long long src0_gap,
                                   const chd_perm_src *srcs, int num_src,
                                   int num_limbs, void *stream) {
  if (!t || !m || !dst || (num_src > 0 && !srcs) || num_polys < 1 ||
      num_polys > CHD_MAX_POLY || num_src < 0 || num_src > CHD_MAX_ACCUM ||
      (num_src == 0 && !src0) || num_limbs < 0)
    return set_error(CHD_ERR_ARG, "chd_k_permute_accum: invalid argument");
  if (num_limbs == 0) return 0;
  PermAccArgs a{};
  for (int p = 0; p < num_polys; p++) {
    if (!dst[p] || (src0 && !src0[p]))
      return set_error(CHD_ERR_ARG, "chd_k_permute_accum: null polynomial");
    a.dst[p] = dst[p];
    a.src0[p] = src0 ? src0[p] : nullptr;
  }
  a.src0_gap = src0_gap;
  for (int j = 0; j < num_src; j++) {
    for (int p = 0; p < num_polys; p++)
      if (!srcs[j].src[p])
        return set_error(CHD_ERR_ARG, "chd_k_permute_accum: null source");
    if ((srcs[j].galois & 1u) == 0 || srcs[j].galois >= 2u * kN)
      return set_error(CHD_ERR_ARG, "chd_k_permute_accum: invalid galois factor");
    a.s[j] = srcs[j];
  }
  dim3 g(kN / kCoefPerBlock, num_limbs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (num_polys) {
    case 1:
      hipLaunchKernelGGL(permute_accum_kernel<1>, g, dim3(kThreads), 0, s, *t, *m, a, num_src);
      break;
    case 2:
      hipLaunchKernelGGL(permute_accum_kernel<2>, g, dim3(kThreads), 0, s, *t, *m, a, num_src);
      break;
    default:
      hipLaunchKernelGGL(permute_accum_kernel<3>, g, dim3(kThreads), 0, s, *t, *m, a, num_src);
      break;
  }
  return check_launch("chd_k_permute_accum");
}

extern "C" int chd_k_bs_fused(const chd_tables *t, const chd_limb_map *m,
                              const chd_bs_args *args, void *stream) {
  if (!t || !m || !args || args->num_rot < 1 || args->num_rot > CHD_MAX_BS ||
      args->beta > CHD_MAX_BS_GROUPS ||
      !groups_valid(args->beta, args->alpha, args->group_shift,
                    args->num_q) ||
      !args->modup || !args->d ||
      !args->ct_b || !args->p_prod || args->num_q != m->num_q ||
      m->skip_len != 0)
    return set_error(CHD_ERR_ARG, "chd_k_bs_fused: invalid argument");
  for (int k = 0; k < args->num_rot; k++) {
    if (!args->dst_b[k] || !args->dst_a[k] || (args->galois[k] & 1u) == 0 ||
        args->galois[k] >= 2u * kN)
      return set_error(CHD_ERR_ARG, "chd_k_bs_fused: invalid rotation");
    for (int g = 0; g < args->beta; g++)
      if (!args->kb[k][g] || !args->ka[k][g])
        return set_error(CHD_ERR_ARG, "chd_k_bs_fused: null key pointer");
  }
  dim3 g(kN / kCoefPerBlock, args->num_q + args->alpha);
  hipLaunchKernelGGL(bs_fused_kernel, g, dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), *t, *m, *args);
  return check_launch("chd_k_bs_fused");
}

extern "C" int chd_k_zero(uint32_t *dst, long long words, void *stream) {
  if (!dst || words < 0 || (words & 3) != 0 ||
      (reinterpret_cast<uintptr_t>(dst) & 15) != 0)
    return set_error(CHD_ERR_ARG, "chd_k_zero: invalid argument");
  if (words == 0) return 0;
  const long long n4 = words / 4;
  hipLaunchKernelGGL(zero_kernel, dim3((n4 + kThreads - 1) / kThreads),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     reinterpret_cast<uint4 *>(dst), n4);
  return check_launch("chd_k_zero");
}

extern "C" int chd_k_gs_fused(const chd_tables *t, const chd_limb_map *m,
                              const chd_gs_args *args, int num_limbs,
                              void *stream) {
  if (!t || !m || !args || args->num_bs < 1 ||
      args->num_bs > CHD_GS_MAX_BS || args->num_gs < 1 ||
      args->num_gs > CHD_GS_MAX_GS || num_limbs < 0 || m->skip_len != 0)
    return set_error(CHD_ERR_ARG, "chd_k_gs_fused: invalid argument");
  for (int b = 0; b < args->num_bs; b++)
    if (!args->bs_b[b] || !args->bs_a[b])
      return set_error(CHD_ERR_ARG, "chd_k_gs_fused: null baby step");
  for (int g = 0; g < args->num_gs; g++)
    if (!args->dst_b[g] || !args->dst_a[g])
      return set_error(CHD_ERR_ARG, "chd_k_gs_fused: null destination");
  if (num_limbs == 0) return 0;
  dim3 g(kN / kCoefPerBlock, num_limbs);
  hipLaunchKernelGGL(gs_fused_kernel, g, dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), *t, *m, *args);
  return check_launch("chd_k_gs_fused");
}

extern "C" int chd_k_gs_fused_wide(const chd_tables *t, const chd_limb_map *m,
                                   const chd_gs_wide_args *args, int num_limbs,
                                   void *stream) {
  if (!t || !m || !args || !args->pt_table || args->num_bs < 1 ||
      args->num_bs > CHD_GS_MAX_BS || args->num_bs % 4 != 0 ||
      args->pt_stride < args->num_bs || num_limbs < 0 || m->skip_len != 0)
    return set_error(CHD_ERR_ARG, "chd_k_gs_fused_wide: invalid argument");
  const int ng = args->num_gs;
  if (ng != 8 && ng != 16 && ng != 24 && ng != 28 && ng != 32)
    return set_error(CHD_ERR_ARG,
                     "chd_k_gs_fused_wide: num_gs must be 8, 16, 24, 28 or 32");
  for (int b = 0; b < args->num_bs; b++)
    if (!args->bs_b[b] || !args->bs_a[b])
      return set_error(CHD_ERR_ARG, "chd_k_gs_fused_wide: null baby step");
  for (int g = 0; g < ng; g++)
    if (!args->dst_b[g] || !args->dst_a[g])
      return set_error(CHD_ERR_ARG, "chd_k_gs_fused_wide: null destination");
  if (args->pt_tiled != nullptr &&
      (args->tiled_rows < 0 || args->tiled_rows > ng))
    return set_error(CHD_ERR_ARG,
                     "chd_k_gs_fused_wide: tiled_rows outside [0, num_gs]");
  if (num_limbs == 0) return 0;
  static_assert(kThreads == 256, "gs_wide_kernel splits giant steps over 4 waves");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool tiled = args->pt_tiled != nullptr;
  // Launches of kGsWideLimbs limbs each (512 workgroups, half of what the
  // GPU holds at once), in stream order: each launch's accumulator writes
  // come at its end instead of interleaving with the reads of workgroups
  // that are still streaming plaintexts (config 5: 14 launches take 1,253
  // us of kernel time against 1,281-1,289 us for one, the evaluation 3.07
  // against 3.13 ms; one limb per launch, 28 launches, 3.33 ms; three and
  // four limbs per launch 3,090-3,100 and 3,083-3,091 us against
  // 3,079-3,086 us for two, four A/B rounds in one call). A limb
  // range [a0, a0 + n) is the caller's map (skip_len 0, checked above) with
  // the launch's limbs shifted by a0 through its skip fields.
  constexpr int kGsWideLimbs = 2;
  for (int a0 = 0; a0 < num_limbs; a0 += kGsWideLimbs) {
    chd_limb_map mr = *m;
    mr.skip_lo = 0;
    mr.skip_len = a0;
    const dim3 g(kN / (64 * kPerThread),
                 num_limbs - a0 < kGsWideLimbs ? num_limbs - a0 : kGsWideLimbs);
#define CHD_GS_WIDE_LAUNCH(kGw)                                              \
  if (tiled)                                                                 \
    hipLaunchKernelGGL((gs_wide_kernel<kGw, true>), g, dim3(kThreads), 0, s, \
                       *t, mr, *args);                                       \
  else                                                                       \
    hipLaunchKernelGGL((gs_wide_kernel<kGw, false>), g, dim3(kThreads), 0,   \
                       s, *t, mr, *args)
    switch (ng) {
      case 8: CHD_GS_WIDE_LAUNCH(2); break;
      case 16: CHD_GS_WIDE_LAUNCH(4); break;
      case 24: CHD_GS_WIDE_LAUNCH(6); break;
      case 28: CHD_GS_WIDE_LAUNCH(7); break;
      default: CHD_GS_WIDE_LAUNCH(8); break;
    }
#undef CHD_GS_WIDE_LAUNCH
  }
  return check_launch("chd_k_gs_fused_wide");
}

extern "C" int chd_k_gs_pack_tiled(const uint32_t *const *pt_table, int rows,
                                   int pt_stride, int num_limbs, uint32_t *dst,
                                   void *stream) {
  if (!pt_table || !dst || rows < 1 || rows > CHD_GS_WIDE_GS ||
      pt_stride < 1 || pt_stride > CHD_GS_MAX_BS || num_limbs < 0 ||
      num_limbs > 65535)
    return set_error(CHD_ERR_ARG, "chd_k_gs_pack_tiled: invalid argument");
  if (num_limbs == 0) return 0;
  dim3 g(kN >> 8, num_limbs, rows);
  hipLaunchKernelGGL(gs_pack_tiled_kernel, g, dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), pt_table, rows,
                     pt_stride, dst);
  return check_launch("chd_k_gs_pack_tiled");
}

extern "C" int chd_k_gs_untile_row(const uint32_t *tiled, int rows,
                                   int pt_stride, int num_limbs, int g,
                                   int dst_limbs, uint32_t *dst,
                                   void *stream) {
  if (!tiled || !dst || rows < 1 || rows > CHD_GS_WIDE_GS || pt_stride < 1 ||
      pt_stride > CHD_GS_MAX_BS || num_limbs < 0 || num_limbs > 65535 ||
      g < 0 || g >= rows || dst_limbs < 0 || dst_limbs > num_limbs)
    return set_error(CHD_ERR_ARG, "chd_k_gs_untile_row: invalid argument");
  if (dst_limbs == 0) return 0;
  dim3 grid(kN >> 8, dst_limbs);
  hipLaunchKernelGGL(gs_untile_row_kernel, grid, dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), tiled, rows, pt_stride,
                     g, dst_limbs, dst);
  return check_launch("chd_k_gs_untile_row");
}

extern "C" int chd_k_elementwise(const chd_tables *t, const chd_limb_map *m,
                                 const chd_ew_args *args, int num_limbs,
                                 void *stream) {
  if (!t || !m || !args || num_limbs < 1 || args->num_poly < 1 ||
      args->num_poly > CHD_MAX_POLY || args->op < CHD_EW_ADD ||
      args->op > CHD_EW_COPY || m->skip_len != 0)
    return set_error(CHD_ERR_ARG, "chd_k_elementwise: invalid argument");
  const int op = args->op;
  const bool need_b =
      op == CHD_EW_ADD || op == CHD_EW_SUB || op == CHD_EW_MULT;
  const bool need_c = op >= CHD_EW_ADD_CONST && op <= CHD_EW_MULT_CONST;
  if ((need_c && !args->cst) || (op == CHD_EW_PMULT && !args->b[0]))
    return set_error(CHD_ERR_ARG, "chd_k_elementwise: missing operand");
  for (int p = 0; p < args->num_poly; p++)
    if (!args->dst[p] || !args->a[p] || (need_b && !args->b[p]))
      return set_error(CHD_ERR_ARG, "chd_k_elementwise: null polynomial");
  dim3 g(kN / kCoefPerBlock, num_limbs);
  hipLaunchKernelGGL(elementwise_kernel, g, dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), *t, *m, *args);
  return check_launch("chd_k_elementwise");
}
