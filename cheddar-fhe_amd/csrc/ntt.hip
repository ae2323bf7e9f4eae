// Negacyclic NTT / INTT for N = 2^16 on gfx950.
//
// Two layouts of the same transform:
// - Two passes (any call, in place included): four-step split N = 256 rows
//   x 256 columns (index = row*256 + col). Forward Cooley-Tukey stages 0..7
//   pair rows (a column pass), stages 8..15 pair columns inside one row (a
//   row pass); each pass is one kernel, one HBM read and one HBM write of
//   every limb. Inside a pass a thread holds 16 elements in registers, runs
//   4 radix-2 stages on them, exchanges through LDS, and runs the next 4.
// - Single pass (forward, source apart from destination): four workgroups
//   per limb, one per output quarter, one HBM read and one HBM write of the
//   limb (ntt_fwd_1p below).
//
// Semantics follow the reference exactly (bit-exact canonical outputs):
//   forward: y[i] = sum_j x_j psi^{(2 brev(i)+1) j}, twiddle psi_rev[m+i]
//            (Montgomery form) for butterfly group i of the stage with m
//            groups (include/core/NTTUtils.cuh:19-34, 62-87;
//            src/core/NTT.cu:231-454)
//   inverse: Gentleman-Sande with psi_inv_rev[m+i], computes N*intt; the
//            N^-1 and any per-limb factor live in the epilogue constant,
//            applied as MontMul(x, c) (NTT.cu:23-229, 673-813).
// Arithmetic. Primes below 2^30 use unsigned lazy butterflies whose
// Montgomery product is the 64-bit multiply-add form (three instructions,
// mont_mad); primes in [2^30, 2^31) use the reference's signed lazy
// butterfly (NTTUtils.cuh:19-60) in Montgomery-Shoup form, MontMul(b, w) =
// mulhi(b, w) - mulhi(b w' mod 2^32, q) with w' = w q^-1. The per-twiddle
// companion (w (-q^-1) or w q^-1) is derived on the fly: one multiply per
// twiddle, scalar when the twiddle is wave-uniform.
#include <algorithm>
#include <type_traits>

#include "chd_device.h"
#include "kernel_common.h"
#include "ntt.h"
#include "overlap.h"

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

// (b * w * 2^-32) mod q in (-q, q) for |b w| < q 2^31 (Basic.cuh:72-137)
__device__ __forceinline__ int32_t mont(int32_t b, int32_t w, int32_t wq,
                                        int32_t q) {
  int32_t hi = __mulhi(b, w);
  int32_t t = static_cast<int32_t>(static_cast<uint32_t>(b) *
                                   static_cast<uint32_t>(wq));
  return hi - __mulhi(t, q);
}

// the same for a per-lane twiddle, without the companion w q^-1: b w as one
// 64-bit product (v_mad_i64_i32), t = (b w mod 2^32) q^-1
__device__ __forceinline__ int32_t mont_s(int32_t b, int32_t w, uint32_t qinv,
                                          int32_t q) {
  const int64_t p = static_cast<int64_t>(b) * w;
  const int32_t t =
      static_cast<int32_t>(static_cast<uint32_t>(p) * qinv);
  return static_cast<int32_t>(p >> 32) - __mulhi(t, q);
}

// [-q, q) -> [0, q) with one add and an unsigned min
__device__ __forceinline__ int32_t norm(int32_t a, int32_t q) {
  uint32_t ua = static_cast<uint32_t>(a);
  uint32_t uq = ua + static_cast<uint32_t>(q);
  return static_cast<int32_t>(ua < uq ? ua : uq);
}

// ButterflyNTT (NTTUtils.cuh:19-34): a, b in [-q, q); m = MontMul(b, w)
__device__ __forceinline__ void ct_bfly_m(int32_t &a, int32_t &b, int32_t m,
                                          int32_t q) {
  m = norm(m, q);
  int32_t an = norm(a, q);
  b = an - m;
  a = (an - q) + m;
}
__device__ __forceinline__ void ct_bfly(int32_t &a, int32_t &b, int32_t w,
                                        int32_t wq, int32_t q) {
  ct_bfly_m(a, b, mont(b, w, wq, q), q);
}

// ButterflyINTT (NTTUtils.cuh:46-60); returns an - bn for the product
__device__ __forceinline__ int32_t gs_bfly_sum(int32_t &a, int32_t b,
                                               int32_t q) {
  int32_t an = norm(a, q);
  int32_t bn = norm(b, q);
  a = (an - q) + bn;
  return an - bn;
}
__device__ __forceinline__ void gs_bfly(int32_t &a, int32_t &b, int32_t w,
                                        int32_t wq, int32_t q) {
  b = mont(gs_bfly_sum(a, b, q), w, wq, q);
}

// Lazy butterflies for q < 2^30 (4q < 2^32), unsigned values: CT keeps
// [0, 4q) (Harvey), GS keeps [0, 2q). The Montgomery product uses the
// 64-bit multiply-add, which gfx950 issues at nearly the full VALU rate: for
// b < 2^32, w < q and wn = w (-q^-1) mod 2^32,
//   d = (b w + (b wn mod 2^32) q) / 2^32  (exact; b w 2^-32 mod q, in [0, 2q))
// is three instructions (v_mad_u64_u32, v_mul_lo_u32, v_mad_u64_u32).
__device__ __forceinline__ uint32_t umin(uint32_t a, uint32_t b) {
  return a < b ? a : b;
}

__device__ __forceinline__ uint32_t mont_mad(uint32_t b, uint32_t w,
                                             uint32_t wn, uint32_t q) {
  const uint64_t t = static_cast<uint64_t>(b) * w;
  const uint32_t m = b * wn;
  return static_cast<uint32_t>((static_cast<uint64_t>(m) * q + t) >> 32);
}

// The same product for a per-lane twiddle: m = (b w mod 2^32) qn equals
// b wn mod 2^32, so no companion of w is needed (the multiply waits for the
// low word of b w instead of running beside it).
__device__ __forceinline__ uint32_t mont_lo(uint32_t b, uint32_t w,
                                            uint32_t qn, uint32_t q) {
  const uint64_t t = static_cast<uint64_t>(b) * w;
  const uint32_t m = static_cast<uint32_t>(t) * qn;
  return static_cast<uint32_t>((static_cast<uint64_t>(m) * q + t) >> 32);
}

// |x - y| + z in one v_sad_u32 (full VALU rate on gfx950). With x >= y it
// is x - y + z, which otherwise takes a subtract and an add. Written as an
// instruction: with a wave-uniform x the compiler expands the max - min + z
// pattern into four instructions instead.
__device__ __forceinline__ uint32_t sad(uint32_t x, uint32_t y, uint32_t z) {
  uint32_t r;
  asm("v_sad_u32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(y), "v"(z));
  return r;
}

// CT: a, b in [0, 4q) -> a + d, a + 2q - d with a reduced to [0, 2q)
// (kRed false: the caller knows a < 2q already). d = b w 2^-32 in [0, 2q).
template <bool kRed = true>
__device__ __forceinline__ void ct_lazy_d(uint32_t &a, uint32_t &b,
                                          uint32_t d, uint32_t q) {
  const uint32_t ar = kRed ? umin(a, a - 2 * q) : a;  // [0, 2q)
  b = sad(2 * q, d, ar);                             // (0, 4q)
  a = ar + d;                                        // [0, 4q)
}
template <bool kRed = true>
__device__ __forceinline__ void ct_lazy(uint32_t &a, uint32_t &b, uint32_t w,
                                        uint32_t wn, uint32_t q) {
  ct_lazy_d<kRed>(a, b, mont_mad(b, w, wn, q), q);
}

// GS: a, b in [0, 2q) -> a + b (reduced), (a - b) w
__device__ __forceinline__ uint32_t gs_lazy_sum(uint32_t &a, uint32_t b,
                                                uint32_t q) {
  const uint32_t s = a + b;                  // [0, 4q)
  const uint32_t t = sad(2 * q, b, a);       // a + 2q - b in (0, 4q)
  a = umin(s, s - 2 * q);                    // [0, 2q)
  return t;
}
__device__ __forceinline__ void gs_lazy(uint32_t &a, uint32_t &b, uint32_t w,
                                        uint32_t wn, uint32_t q) {
  b = mont_mad(gs_lazy_sum(a, b, q), w, wn, q);  // [0, 2q)
}

// [0, 4q) -> [0, q)
__device__ __forceinline__ uint32_t canon4(uint32_t x, uint32_t q) {
  x = umin(x, x - 2 * q);
  return umin(x, x - q);
}

__device__ __forceinline__ int pidx(int i) { return i + (i >> 4); }

// orders a wave's LDS writes before its later LDS reads of the same words
// written by other lanes of that wave: a wave's LDS instructions execute in
// program order, so only the compiler has to be kept from reordering them
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Coalesced tile layout of the row passes: a workgroup owns kTileRows
// consecutive rows (16 KiB contiguous); in store round v (0..3) thread t owns
// the 16 bytes at tile offset 16 (t + 256 v), i.e. tile elements
// 4 (t + 256 v) .. + 3.
__device__ __forceinline__ uint32_t tile_byte(int tile) {
  return static_cast<uint32_t>(tile) * (kTileRows * kCols * 4u);
}
__device__ __forceinline__ uint32_t tile_lane_byte(int v) {
  return (threadIdx.x + 256u * v) * 16u;
}

// base of polynomial z: explicit list or base + z * stride
__device__ __forceinline__ uint32_t *poly_dst(const NttArgs &a, int z) {
  return a.dst_list[0] != nullptr ? a.dst_list[z] : a.dst + z * a.dst_pstride;
}

// Element load/store at a 32-bit byte offset from a wave-uniform base, so the
// compiler emits the scalar-base + 32-bit-offset addressing form.
template <typename T>
__device__ __forceinline__ T ld_at(const void *base, uint32_t byte_off) {
  return *reinterpret_cast<const T *>(static_cast<const char *>(base) +
                                      byte_off);
}
template <typename T>
__device__ __forceinline__ void st_at(void *base, uint32_t byte_off, T v) {
  *reinterpret_cast<T *>(static_cast<char *>(base) + byte_off) = v;
}
// Streaming (nontemporal) variants for limb data that a transform touches
// once: the column passes' loads and stores (whole 128-byte lines per wave
// instruction) and the row passes' strided dword accesses. Measured 8-11%
// faster per transform. The fused key-accumulation kernel keeps default
// loads: with many concurrent streams the hint evicts a half-used line before
// the next instruction reads its other half (twice the traffic, measured).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Wave-uniform read of a table no kernel writes (twiddles, constants): through
// the constant address space it becomes a scalar load into an SGPR instead
// of a vector load plus v_readfirstlane.
typedef const __attribute__((address_space(4))) uint32_t cu32;
__device__ __forceinline__ uint32_t ld_uniform(const uint32_t *p, int i) {
  return ((cu32 *)p)[i];
}
template <typename T>
__device__ __forceinline__ T ld_nt(const void *base, uint32_t byte_off) {
  const char *p = static_cast<const char *>(base) + byte_off;
  if constexpr (sizeof(T) == 16) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    T r;
    __builtin_memcpy(&r, &v, 16);
    return r;
  } else {
    return __builtin_nontemporal_load(reinterpret_cast<const T *>(p));
  }
}
template <typename T>
__device__ __forceinline__ void st_nt(void *base, uint32_t byte_off, T v) {
  __builtin_nontemporal_store(
      v, reinterpret_cast<T *>(static_cast<char *>(base) + byte_off));
}

// Buffer-resource loads (raw buffer, stride 0): address = base + soffset
// (an SGPR) + voffset (a VGPR) + a 12-bit immediate, so a load whose
// per-lane part repeats costs no VALU address arithmetic; the scalar part is
// formed by SALU. The range (bytes) is checked by the hardware: loads beyond
// it return 0. Word 3 0x00020000 is the gfx9 dword data format. Cache policy
// kAux: 0 default, 2 nontemporal.
// Loads only: a buffer store of more than 8 bytes with an SGPR soffset reads
// its data VGPRs after the next instructions have issued, and the compiler
// inserts no wait state for that form (it does for global stores). On gfx950
// a VALU write of the data registers right after such a store put the new
// value into memory under load (measured: the next round's index in the
// first word of a 16-byte output). Stores stay global stores.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0,
                                           static_cast<int>(bytes),
                                           0x00020000);
}
template <int kAux = 0>
__device__ __forceinline__ uint32_t bld1(rsrc_t r, uint32_t voff,
                                         uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, kAux);
}
template <int kAux = 0>
__device__ __forceinline__ u32x2 bld2(rsrc_t r, uint32_t voff,
                                      uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kAux);
}
template <int kAux = 0>
__device__ __forceinline__ u32x4 bld4(rsrc_t r, uint32_t voff,
                                      uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kAux);
}


// the 4 words of store round v (tile_lane_byte) from the padded LDS tile
// (rows of kRowPad words, column i at pidx(i))
__device__ __forceinline__ u32x4 tile_lds4(const uint32_t *xt, int v) {
  const int e = 4 * (threadIdx.x + 256 * v);
  const uint32_t *p = xt + (e >> 8) * kRowPad;
  const int cc = e & 255;
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; j++) o[j] = p[pidx(cc + j)];
  return o;
}

// Per-limb arithmetic policy. Values between the two passes of a transform
// stay unreduced in the policy's range: [0, 4q) (forward, lazy), [0, 2q)
// (inverse, lazy) or [-q, q) (reference form, any q < 2^31).
template <bool kLazy>
struct Arith;

// twq(w) is the per-twiddle companion of w that ct / gs / mul take:
// w (-q^-1) for the lazy form, w q^-1 for the reference form. Wave-uniform
// twiddles use it (a scalar multiply); per-lane twiddles use ctv / gsv,
// which derive the Montgomery factor from the product instead.
// ct<false> skips the reduction of a, for a known to lie in [0, 2q).
template <>
struct Arith<true> {
  using T = uint32_t;
  uint32_t q;
  uint32_t qn;  // -q^-1 mod 2^32
  __device__ Arith(uint32_t q_, uint32_t qinv) : q(q_), qn(0u - qinv) {}
  __device__ uint32_t twq(uint32_t w) const { return w * qn; }
  template <bool kRed = true>
  __device__ void ct(T &a, T &b, uint32_t w, uint32_t wn) const {
    ct_lazy<kRed>(a, b, w, wn, q);
  }
  template <bool kRed = true>
  __device__ void ctv(T &a, T &b, uint32_t w) const {
    ct_lazy_d<kRed>(a, b, mont_lo(b, w, qn, q), q);
  }
  __device__ void gs(T &a, T &b, uint32_t w, uint32_t wn) const {
    gs_lazy(a, b, w, wn, q);
  }
  __device__ void gsv(T &a, T &b, uint32_t w) const {
    b = mont_lo(gs_lazy_sum(a, b, q), w, qn, q);
  }
  // MontMul(x, c) for any representable input, result in [0, 2q)
  __device__ T mul(T x, uint32_t c, uint32_t cn) const {
    return mont_mad(x, c, cn, q);
  }
  __device__ uint32_t canon_fwd(T x) const { return canon4(x, q); }
  __device__ uint32_t canon_inv(T x) const { return umin(x, x - q); }
};

template <>
struct Arith<false> {
  using T = int32_t;
  int32_t q;
  uint32_t qinv;
  __device__ Arith(uint32_t q_, uint32_t qinv_)
      : q(static_cast<int32_t>(q_)), qinv(qinv_) {}
  __device__ uint32_t twq(uint32_t w) const { return w * qinv; }
  template <bool kRed = true>
  __device__ void ct(T &a, T &b, uint32_t w, uint32_t wq) const {
    ct_bfly(a, b, static_cast<int32_t>(w), static_cast<int32_t>(wq), q);
  }
  template <bool kRed = true>
  __device__ void ctv(T &a, T &b, uint32_t w) const {
    ct_bfly_m(a, b, mont_s(b, static_cast<int32_t>(w), qinv, q), q);
  }
  __device__ void gs(T &a, T &b, uint32_t w, uint32_t wq) const {
    gs_bfly(a, b, static_cast<int32_t>(w), static_cast<int32_t>(wq), q);
  }
  __device__ void gsv(T &a, T &b, uint32_t w) const {
    b = mont_s(gs_bfly_sum(a, b, q), static_cast<int32_t>(w), qinv, q);
  }
  __device__ T mul(T x, uint32_t c, uint32_t cq) const {
    return mont(x, static_cast<int32_t>(c), static_cast<int32_t>(cq), q);
  }
  __device__ uint32_t canon_fwd(T x) const {
    return static_cast<uint32_t>(norm(x, q));
  }
  __device__ uint32_t canon_inv(T x) const {
    return static_cast<uint32_t>(norm(x, q));
  }
};

// ------------------------------------------------------------------------
// Kernel skeleton: each kernel decodes its limb, issues the data loads of the
// whole tile first (they depend on kernel arguments only), then reads the
// prime and twiddles and branches to the lazy (q < 2^30) or reference-form
// body. Twiddles of both half-passes are fetched before the LDS barrier.
// ------------------------------------------------------------------------

// forward, column pass: stages 0..7 (src -> dst, dst left unreduced)
// grid (kCols / kTileCols, limbs, polys), block 512
template <bool kPre, bool kLazy>
__device__ __forceinline__ void fwd_cols_body(const NttArgs &a, const Limb &lb,
                                              uint32_t (&xin)[16], uint32_t q,
                                              uint32_t qinv, void *dst,
                                              int32_t *xch) {
  using A = Arith<kLazy>;
  using T = typename A::T;
  const A ar(q, qinv);
  const uint32_t *tw = a.tab.tw + (static_cast<size_t>(lb.ti) << kLogN);
  const int c = threadIdx.x & (kTileCols - 1);
  const int rg = threadIdx.x / kTileCols;  // 0..15
  const uint32_t col = blockIdx.x * kTileCols + c;
  uint32_t w2[15];
#pragma unroll
  for (int s = 4, i = 0; s < 8; s++)
#pragma unroll
    for (int g = 0; g < (1 << (s - 4)); g++, i++)
      w2[i] = tw[(1 << s) + (rg << (s - 4)) + g];

  T x[16];
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = static_cast<T>(xin[k]);
  if constexpr (kPre) {
    const uint32_t ce = a.cst[lb.ci];
    const uint32_t ceq = ar.twq(ce);
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = ar.mul(x[k], ce, ceq);
  }
  // stages 0..3: rows rg + 16k, twiddles identical for every thread
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const int h = 8 >> s;
#pragma unroll
    for (int g = 0; g < (1 << s); g++) {
      const uint32_t w = ld_uniform(tw, (1 << s) + g);
      const uint32_t wq = ar.twq(w);
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++) ar.ct(x[k], x[k + h], w, wq);
    }
  }
  T *xt = reinterpret_cast<T *>(xch);
#pragma unroll
  for (int k = 0; k < 16; k++) xt[(rg + 16 * k) * kTileCols + c] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = xt[(16 * rg + k) * kTileCols + c];
  // stages 4..7: rows 16 rg + k
#pragma unroll
  for (int s = 4, i = 0; s < 8; s++) {
    const int h = 8 >> (s - 4);
#pragma unroll
    for (int g = 0; g < (1 << (s - 4)); g++, i++) {
      const uint32_t w = w2[i];  // per lane
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++) ar.ctv(x[k], x[k + h], w);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; k++)
    st_nt<T>(dst, ((16 * rg + k) * kCols + col) * 4u, x[k]);
}

template <bool kPre>
__global__ __launch_bounds__(512) void ntt_fwd_cols(NttArgs a) {
  __shared__ int32_t xch[kRows * kTileCols];
  LimbMap m = a.map;
  if (a.group_alpha > 0) {
    const int g = a.group_period > 0 ? static_cast<int>(blockIdx.z) % a.group_period
                                     : static_cast<int>(blockIdx.z);
    m.skip_lo = group_lo(g, a.group_alpha, a.group_shift);
    m.skip_len =
        group_hi(g, a.group_alpha, a.group_shift, m.num_q) - m.skip_lo;
    if (static_cast<int>(blockIdx.y) >= a.group_limbs - m.skip_len) return;
  }
  const Limb lb = decode(m, blockIdx.y);
  const uint32_t *sbase =
      a.dst_list[0] != nullptr ? a.dst_list[blockIdx.z]
                               : a.src + blockIdx.z * a.src_pstride;
  const void *src = sbase + (static_cast<size_t>(lb.sl) << kLogN);
  void *dst =
      poly_dst(a, blockIdx.z) + (static_cast<size_t>(lb.l) << kLogN);
  const uint32_t col = blockIdx.x * kTileCols + (threadIdx.x & (kTileCols - 1));
  const int rg = threadIdx.x / kTileCols;
  uint32_t x[16];
#pragma unroll
  for (int k = 0; k < 16; k++)
    x[k] = ld_nt<uint32_t>(src, ((rg + 16 * k) * kCols + col) * 4u);
  const uint32_t q = a.tab.q[lb.ti];
  const uint32_t qinv = static_cast<uint32_t>(a.tab.qinv[lb.ti]);
  if (q < (1u << 30))
    fwd_cols_body<kPre, true>(a, lb, x, q, qinv, dst, xch);
  else
    fwd_cols_body<kPre, false>(a, lb, x, q, qinv, dst, xch);
}

// forward, row pass: stages 8..15 (in place on dst) + epilogue
// grid (kRows / kTileRows, limbs, polys), block 256
template <int kEpi, bool kLazy>
__device__ __forceinline__ void fwd_rows_body(const NttArgs &a, const Limb &lb,
                                              uint32_t (&xin)[16], uint32_t q,
                                              uint32_t qinv, uint32_t *dst,
                                              int32_t *xch,
                                              const uint32_t (&s2v)[16]) {
  using A = Arith<kLazy>;
  using T = typename A::T;
  const A ar(q, qinv);
  const uint32_t *tw = a.tab.tw + (static_cast<size_t>(lb.ti) << kLogN);
  const int c = threadIdx.x & 15;
  const int r = threadIdx.x >> 4;
  const int row = blockIdx.x * kTileRows + r;
  T *xr = reinterpret_cast<T *>(xch) + r * kRowPad;
  uint32_t w1[15], w2[15];
#pragma unroll
  for (int s = 0, i = 0; s < 4; s++)
#pragma unroll
    for (int g = 0; g < (1 << s); g++, i++) {
      w1[i] = tw[(256 << s) + (row << s) + g];
      w2[i] = tw[(4096 << s) + (row << (4 + s)) + (c << s) + g];
    }

  T x[16];
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = static_cast<T>(xin[k]);
  // stages 8..11: columns c + 16k, twiddles depend on the row only
#pragma unroll
  for (int s = 0, i = 0; s < 4; s++) {
    const int h = 8 >> s;
#pragma unroll
    for (int g = 0; g < (1 << s); g++, i++) {
      const uint32_t w = w1[i];  // per lane
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++) ar.ctv(x[k], x[k + h], w);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; k++) xr[pidx(c + 16 * k)] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = xr[pidx(16 * c + k)];
  // stages 12..15: columns 16c + k
#pragma unroll
  for (int s = 0, i = 0; s < 4; s++) {
    const int h = 8 >> s;
#pragma unroll
    for (int g = 0; g < (1 << s); g++, i++) {
      const uint32_t w = w2[i];  // per lane
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++) ar.ctv(x[k], x[k + h], w);
    }
  }
  // canonical values back through LDS: each wave then stores 1 KiB of the
  // tile's contiguous 16 KiB per instruction (a lane's own 16 words would
  // be 16-byte pieces at a 64-byte stride, four times the cache lines per
  // store instruction)
  __syncthreads();  // every lane has read its exchange values
  uint32_t *xu = reinterpret_cast<uint32_t *>(xr);
#pragma unroll
  for (int k = 0; k < 16; k++) xu[pidx(16 * c + k)] = ar.canon_fwd(x[k]);
  __syncthreads();
  const uint32_t *xt = reinterpret_cast<const uint32_t *>(xch);
  char *tile = reinterpret_cast<char *>(dst) + tile_byte(blockIdx.x);
  [[maybe_unused]] const int32_t qs = static_cast<int32_t>(q);
  [[maybe_unused]] int32_t c2 = 0, c2q = 0;
  if constexpr (kEpi == kEpiModDown) {
    c2 = static_cast<int32_t>(a.cst2[lb.l]);
    c2q = static_cast<int32_t>(static_cast<uint32_t>(c2) * qinv);
  }
#pragma unroll
  for (int v = 0; v < 4; v++) {
    u32x4 o = tile_lds4(xt, v);
    if constexpr (kEpi == kEpiModDown) {
      // NTTPhase2ForModDown epilogue (NTT.cu:567-600); src2 (and its
      // optional padding product) was loaded before the butterflies
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int32_t d = static_cast<int32_t>(s2v[4 * v + j]) -
                          static_cast<int32_t>(o[j]);
        o[j] = static_cast<uint32_t>(norm(mont(d, c2, c2q, qs), qs));
      }
    }
    st_nt<u32x4>(tile, tile_lane_byte(v), o);
  }
}

template <int kEpi>
__global__ __launch_bounds__(256) void ntt_fwd_rows(NttArgs a) {
  __shared__ int32_t xch[kTileRows * kRowPad];
  LimbMap m = a.map;
  if (a.group_alpha > 0) {
    const int g = a.group_period > 0 ? static_cast<int>(blockIdx.z) % a.group_period
                                     : static_cast<int>(blockIdx.z);
    m.skip_lo = group_lo(g, a.group_alpha, a.group_shift);
    m.skip_len =
        group_hi(g, a.group_alpha, a.group_shift, m.num_q) - m.skip_lo;
    if (static_cast<int>(blockIdx.y) >= a.group_limbs - m.skip_len) return;
  }
  const Limb lb = decode(m, blockIdx.y);
  uint32_t *dst =
      poly_dst(a, blockIdx.z) + (static_cast<size_t>(lb.l) << kLogN);
  const int c = threadIdx.x & 15;
  const uint32_t rbase =
      static_cast<uint32_t>((blockIdx.x * kTileRows + (threadIdx.x >> 4)) *
                            kCols) * 4u;
  uint32_t x[16];
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = ld_nt<uint32_t>(dst, rbase + (c + 16 * k) * 4u);
  // ModDown epilogue operand: src2 at this thread's 16 output words of the
  // coalesced store layout (zero outside [src2_lo, src2_hi)), loaded with the
  // data so their latency hides behind the butterflies
  uint32_t s2v[16] = {};
  if constexpr (kEpi == kEpiModDown) {
    if (lb.l >= a.src2_lo && lb.l < a.src2_hi) {
      const uint32_t *s2p = a.src2 + blockIdx.z * a.src2_pstride +
                            (static_cast<size_t>(lb.l - a.src2_lo) << kLogN);
      const char *s2t = reinterpret_cast<const char *>(s2p) +
                        tile_byte(blockIdx.x);
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const uint4 t = ld_nt<uint4>(s2t, tile_lane_byte(v));
        s2v[4 * v] = t.x;
        s2v[4 * v + 1] = t.y;
        s2v[4 * v + 2] = t.z;
        s2v[4 * v + 3] = t.w;
      }
    }
  }
  const uint32_t q = a.tab.q[lb.ti];
  const uint32_t qinv = static_cast<uint32_t>(a.tab.qinv[lb.ti]);
  if constexpr (kEpi == kEpiModDown) {
    if (a.pad != nullptr && lb.l >= a.src2_lo && lb.l < a.src2_hi) {
      // src2 * padding (BitPacker restore, NTT.cu:579-585)
      const int32_t qs = static_cast<int32_t>(q);
      const int32_t pe = static_cast<int32_t>(a.pad[lb.l - a.src2_lo]);
      const int32_t peq = static_cast<int32_t>(static_cast<uint32_t>(pe) * qinv);
#pragma unroll
      for (int k = 0; k < 16; k++)
        s2v[k] = static_cast<uint32_t>(
            norm(mont(static_cast<int32_t>(s2v[k]), pe, peq, qs), qs));
    }
  }
  if (q < (1u << 30))
    fwd_rows_body<kEpi, true>(a, lb, x, q, qinv, dst, xch, s2v);
  else
    fwd_rows_body<kEpi, false>(a, lb, x, q, qinv, dst, xch, s2v);
}

// twiddles of the inverse row pass for this thread of a 16-row tile (row
// tile blockIdx.x): w2 for stages 15..12 (columns 16c + k), w1 for stages
// 11..8 (the row's)
__device__ __forceinline__ void inv_row_twiddles(const uint32_t *itw,
                                                 uint32_t (&w1)[15],
                                                 uint32_t (&w2)[15]) {
  const int c = threadIdx.x & 15;
  const int row = blockIdx.x * kTileRows + (threadIdx.x >> 4);
#pragma unroll
  for (int s = 0, i = 0; s < 4; s++)
#pragma unroll
    for (int g = 0; g < (1 << s); g++, i++) {
      w2[i] = itw[(4096 << s) + (row << (4 + s)) + (c << s) + g];
      w1[i] = itw[(256 << s) + (row << s) + g];
    }
}

// inverse, row pass: GS stages 15..8 of this workgroup's 16-row tile (row
// tile blockIdx.x) with the limb's inverse twiddles tw; xin holds columns
// 16c .. 16c+15 of the thread's row; dst (the limb) is left unreduced.
template <bool kLazy>
__device__ __forceinline__ void inv_rows_body(const uint32_t (&w1)[15],
                                              const uint32_t (&w2)[15],
                                              uint32_t (&xin)[16], uint32_t q,
                                              uint32_t qinv, uint32_t *dst,
                                              int32_t *xch) {
  using A = Arith<kLazy>;
  using T = typename A::T;
  const A ar(q, qinv);
  const int c = threadIdx.x & 15;
  const int r = threadIdx.x >> 4;
  T *xr = reinterpret_cast<T *>(xch) + r * kRowPad;
  T x[16];
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = static_cast<T>(xin[k]);
  // stages 15..12: columns 16c + k
#pragma unroll
  for (int s = 3; s >= 0; s--) {
    const int h = 8 >> s;
#pragma unroll
    for (int g = 0; g < (1 << s); g++) {
      const uint32_t w = w2[(1 << s) - 1 + g];  // per lane
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++) ar.gsv(x[k], x[k + h], w);
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
      const uint32_t w = w1[(1 << s) - 1 + g];  // per lane
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++) ar.gsv(x[k], x[k + h], w);
    }
  }
  // through LDS again so each wave stores 1 KiB contiguous per instruction
  __syncthreads();  // every lane has read its exchange values
#pragma unroll
  for (int k = 0; k < 16; k++) xr[pidx(c + 16 * k)] = x[k];
  __syncthreads();
  const uint32_t *xt = reinterpret_cast<const uint32_t *>(xch);
  char *tile = reinterpret_cast<char *>(dst) + tile_byte(blockIdx.x);
#pragma unroll
  for (int v = 0; v < 4; v++) st_nt<u32x4>(tile, tile_lane_byte(v), tile_lds4(xt, v));
}

__global__ __launch_bounds__(256) void ntt_inv_rows(NttArgs a) {
  __shared__ int32_t xch[kTileRows * kRowPad];
  const Limb lb = decode(a.map, blockIdx.y);
  const uint32_t *src = a.src + blockIdx.z * a.src_pstride +
                        (static_cast<size_t>(lb.sl) << kLogN);
  uint32_t *dst =
      poly_dst(a, blockIdx.z) + (static_cast<size_t>(lb.l) << kLogN);
  const int c = threadIdx.x & 15;
  // the tile (16 contiguous rows) is read with coalesced 16-byte loads and
  // regrouped through LDS into this thread's 16 consecutive columns (1 us
  // faster at 64 limbs than 16-byte loads at a 64-byte stride, measured)
  const char *tile = reinterpret_cast<const char *>(src) + tile_byte(blockIdx.x);
  u32x4 v4[4];
#pragma unroll
  for (int v = 0; v < 4; v++) v4[v] = ld_at<u32x4>(tile, tile_lane_byte(v));
  // twiddles of both half-passes, requested with the tile so their latency
  // hides behind its load and the LDS regrouping (stages 15..12: columns
  // 16c + k; stages 11..8: the row's)
  uint32_t w1[15], w2[15];
  inv_row_twiddles(a.tab.itw + (static_cast<size_t>(lb.ti) << kLogN), w1, w2);
  const uint32_t q = a.tab.q[lb.ti];
  const uint32_t qinv = static_cast<uint32_t>(a.tab.qinv[lb.ti]);
  if (a.src_mul != nullptr) {
    // Tensor's rx = MontMul(a1, a2) (ElementWise.cu:504-546), canonical
    const char *sm = reinterpret_cast<const char *>(
                         a.src_mul + blockIdx.z * a.src_pstride +
                         (static_cast<size_t>(lb.sl) << kLogN)) +
                     tile_byte(blockIdx.x);
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const u32x4 y = ld_at<u32x4>(sm, tile_lane_byte(v));
#pragma unroll
      for (int j = 0; j < 4; j++)
        v4[v][j] = mont_mul(static_cast<int32_t>(v4[v][j]),
                            static_cast<int32_t>(y[j]), q,
                            static_cast<int32_t>(qinv));
    }
  }
  uint32_t *xt = reinterpret_cast<uint32_t *>(xch);
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int e = 4 * (threadIdx.x + 256 * v);
    uint32_t *p = xt + (e >> 8) * kRowPad;
#pragma unroll
    for (int j = 0; j < 4; j++) p[pidx((e & 255) + j)] = v4[v][j];
  }
  __syncthreads();
  // each thread then reads (and later rewrites) only its own 16 words
  const uint32_t *xr = xt + (threadIdx.x >> 4) * kRowPad;
  uint32_t x[16];
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = xr[pidx(16 * c + k)];
  if (q < (1u << 30))
    inv_rows_body<true>(w1, w2, x, q, qinv, dst, xch);
  else
    inv_rows_body<false>(w1, w2, x, q, qinv, dst, xch);
}

// inverse, column pass: GS stages 7..0 (in place on dst) + constant epilogue
// (INTTPhase2 with MultConst / MultConstNormalize, NTTUtils.cuh:369-391)
template <int kEpi, bool kLazy>
__device__ __forceinline__ void inv_cols_body(const NttArgs &a, const Limb &lb,
                                              uint32_t (&xin)[16], uint32_t q,
                                              uint32_t qinv, uint32_t *dst,
                                              int32_t *xch) {
  using A = Arith<kLazy>;
  using T = typename A::T;
  const A ar(q, qinv);
  const uint32_t *tw = a.tab.itw + (static_cast<size_t>(lb.ti) << kLogN);
  const int c = threadIdx.x & (kTileCols - 1);
  const int rg = threadIdx.x / kTileCols;
  const uint32_t col = blockIdx.x * kTileCols + c;
  uint32_t w2[15], w1[15];
#pragma unroll
  for (int s = 4, i = 0; s < 8; s++)
#pragma unroll
    for (int g = 0; g < (1 << (s - 4)); g++, i++)
      w2[i] = tw[(1 << s) + (rg << (s - 4)) + g];
  // the second half's (wave-uniform) twiddles and the epilogue constant,
  // requested now so that no wave waits for them after the barrier
#pragma unroll
  for (int i = 0; i < 15; i++) w1[i] = ld_uniform(tw, 1 + i);
  const uint32_t ce = a.cst[lb.ci];

  T x[16];
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = static_cast<T>(xin[k]);
#pragma unroll
  for (int s = 7; s >= 4; s--) {
    const int h = 8 >> (s - 4);
#pragma unroll
    for (int g = 0; g < (1 << (s - 4)); g++) {
      const uint32_t w = w2[(1 << (s - 4)) - 1 + g];  // per lane
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++) ar.gsv(x[k], x[k + h], w);
    }
  }
  T *xt = reinterpret_cast<T *>(xch);
#pragma unroll
  for (int k = 0; k < 16; k++) xt[(16 * rg + k) * kTileCols + c] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = xt[(rg + 16 * k) * kTileCols + c];
#pragma unroll
  for (int s = 3; s >= 0; s--) {
    const int h = 8 >> s;
#pragma unroll
    for (int g = 0; g < (1 << s); g++) {
      const uint32_t w = w1[(1 << s) - 1 + g];
      const uint32_t wq = ar.twq(w);
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++) ar.gs(x[k], x[k + h], w, wq);
    }
  }
  const uint32_t ceq = ar.twq(ce);
  const int32_t qs = static_cast<int32_t>(q);
#pragma unroll
  for (int k = 0; k < 16; k++) {
    int32_t v = static_cast<int32_t>(ar.canon_inv(ar.mul(x[k], ce, ceq)));
    if constexpr (kEpi == kEpiConstCentre)
      if (v > (qs >> 1)) v -= qs;
    st_nt<int32_t>(dst, ((rg + 16 * k) * kCols + col) * 4u, v);
  }
}

template <int kEpi>
__global__ __launch_bounds__(512) void ntt_inv_cols(NttArgs a) {
  __shared__ int32_t xch[kRows * kTileCols];
  const Limb lb = decode(a.map, blockIdx.y);
  uint32_t *dst =
      poly_dst(a, blockIdx.z) + (static_cast<size_t>(lb.l) << kLogN);
  const uint32_t col = blockIdx.x * kTileCols + (threadIdx.x & (kTileCols - 1));
  const int rg = threadIdx.x / kTileCols;
  uint32_t x[16];
#pragma unroll
  for (int k = 0; k < 16; k++)
    x[k] = ld_nt<uint32_t>(dst, ((16 * rg + k) * kCols + col) * 4u);
  const uint32_t q = a.tab.q[lb.ti];
  const uint32_t qinv = static_cast<uint32_t>(a.tab.qinv[lb.ti]);
  if (q < (1u << 30))
    inv_cols_body<kEpi, true>(a, lb, x, q, qinv, dst, xch);
  else
    inv_cols_body<kEpi, false>(a, lb, x, q, qinv, dst, xch);
}


// ------------------------------------------------------------------------
// Fused ModUp row pass + evk inner product + CAccum (Context.cpp:609-712):
//   acc_{b,a}[l] = sum_g MontMul(u_g[l], key_g.{b,a}[l'])
//                  (+ MontMul(p_prod[l], c{b,a}[l]) for q limbs)
// where u_g[l] = d[l] for the group's own limbs and otherwise the forward
// NTT of BConv output (stages 8..15 done here on the column-pass result).
// The ModUp output never goes back to HBM. grid (kRows/kTileRows, L+alpha).
// ------------------------------------------------------------------------
template <bool kLazy>
__device__ __forceinline__ void keyacc_body(const chd_keyacc_args &a,
                                            const chd_tables &tab, int l,
                                            bool aux, int ti, uint32_t q,
                                            uint32_t qinv, int32_t *xch) {
  using A = Arith<kLazy>;
  using T = typename A::T;
  const A ar(q, qinv);
  const int32_t qs = static_cast<int32_t>(q);
  const int32_t qi = static_cast<int32_t>(qinv);
  const uint32_t *tw = tab.tw + (static_cast<size_t>(ti) << kLogN);
  const int c = threadIdx.x & 15;
  const int r = threadIdx.x >> 4;
  const int row = blockIdx.x * kTileRows + r;
  const uint32_t rbase = static_cast<uint32_t>(row * kCols) * 4u;
  // Element ownership of the products: register k = 4v + j holds column
  // 4c + 64v + j of the thread's row, so the 16 threads of a row move 256
  // contiguous bytes per 16-byte access (keys, CAccum inputs, outputs). A
  // row's 16 threads are lanes of one wave: its LDS exchanges need only a
  // wave-level fence.
  const uint32_t obase = rbase + 16u * c;
  T *xr = reinterpret_cast<T *>(xch) + r * kRowPad;
  // twiddles are (re)loaded inside each group's row pass (cache hits after
  // the first group) instead of living in 30 registers across the loop
  const size_t loff = static_cast<size_t>(l) << kLogN;
  const size_t koff = loff + (aux ? a.key_gap : 0);
  // The inner product and CAccum are sums of products of canonical residues
  // (the reference adds MontMul results, CPAccum in ElementWise.cu:225-287,
  // called from Context.cpp:609-712). Here each
  // product goes into a 64-bit sum with one v_mad_u64_u32; at most four
  // products share a sum (< 4 q^2 < 2^64), which one Montgomery reduction
  // folds into the canonical accumulators: the same residue,
  // sum(a_i b_i) 2^-32 mod q.
  const uint32_t qn = 0u - qinv;
  uint64_t sb[16], sa[16];
  uint32_t accb[16], acca[16];
#pragma unroll
  for (int k = 0; k < 16; k++) {
    sb[k] = sa[k] = 0;
    accb[k] = acca[k] = 0;
  }
  // the ModDown INTT row pass's twiddles of an aux limb, requested before
  // the group loop so that the last phase does not wait for them
  const bool intt_here = a.intt_b != nullptr && l >= a.intt_lo;
  uint32_t iw1[15], iw2[15];
  if (intt_here)
    inv_row_twiddles(tab.itw + (static_cast<size_t>(ti) << kLogN), iw1, iw2);
  int nprod = 0;        // products in sb / sa (uniform)
  bool folded = false;  // accb / acca hold earlier products
  auto fold = [&]() {
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const uint32_t rb = reduce_sum4(sb[k], q, qn);
      const uint32_t ra = reduce_sum4(sa[k], q, qn);
      accb[k] = folded ? add_mod(accb[k], rb, q) : rb;
      acca[k] = folded ? add_mod(acca[k], ra, q) : ra;
      sb[k] = sa[k] = 0;
    }
    folded = true;
    nprod = 0;
  };
  for (int g = 0; g < a.beta; g++) {
    const int own_lo = group_lo(g, a.alpha, a.group_shift);
    const int own_hi = group_hi(g, a.alpha, a.group_shift, a.num_q);
    const bool own = l >= own_lo && l < own_hi;
    // this group adds the key product, and on a tensor-mode own limb the
    // CAccum product as well
    const int np = own && a.a1 != nullptr ? 2 : 1;
    if (nprod + np > 4) fold();
    nprod += np;
    uint32_t u[16];
    if (own) {
      // own limb: the input itself (ModSwitch.cu:466-470 copies it); in
      // tensor mode the input is rx = MontMul(a1, a2), and the CAccum of
      // this q limb (Context.cpp:684-699) is done here too, from the same
      // loads of the two ciphertexts: bx = MontMul(b1, b2),
      // ax = MontMul(b1 - q + a1, b2 - q + a2) - bx - rx (ElementWise.cu:504-546)
      if (a.a1 != nullptr) {
        const uint64_t pp = a.p_prod[l];
#pragma unroll
        for (int v = 0; v < 4; v++) {
          const uint4 vb1 = ld_at<uint4>(a.b1 + loff, obase + 256u * v);
          const uint4 va1 = ld_at<uint4>(a.a1 + loff, obase + 256u * v);
          const uint4 vb2 = ld_at<uint4>(a.b2 + loff, obase + 256u * v);
          const uint4 va2 = ld_at<uint4>(a.a2 + loff, obase + 256u * v);
          const uint32_t x1[4] = {vb1.x, vb1.y, vb1.z, vb1.w};
          const uint32_t y1[4] = {va1.x, va1.y, va1.z, va1.w};
          const uint32_t x2[4] = {vb2.x, vb2.y, vb2.z, vb2.w};
          const uint32_t y2[4] = {va2.x, va2.y, va2.z, va2.w};
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int32_t s1 = (static_cast<int32_t>(x1[j]) - qs) +
                               static_cast<int32_t>(y1[j]);
            const int32_t s2 = (static_cast<int32_t>(x2[j]) - qs) +
                               static_cast<int32_t>(y2[j]);
            const uint32_t bb = mont_mul(static_cast<int32_t>(x1[j]),
                                         static_cast<int32_t>(x2[j]), q, qi);
            const uint32_t rr = mont_mul(static_cast<int32_t>(y1[j]),
                                         static_cast<int32_t>(y2[j]), q, qi);
            const uint32_t ax = sub_mod(
                sub_mod(mont_mul(s1, s2, q, qi), bb, q), rr, q);
            u[4 * v + j] = rr;
            sb[4 * v + j] += pp * bb;
            sa[4 * v + j] += pp * ax;
          }
        }
      } else {
        const uint32_t *dl = a.d + loff;
#pragma unroll
        for (int v = 0; v < 4; v++) {
          uint4 t = ld_at<uint4>(dl, obase + 256u * v);
          u[4 * v] = t.x;
          u[4 * v + 1] = t.y;
          u[4 * v + 2] = t.z;
          u[4 * v + 3] = t.w;
        }
      }
    } else {
      uint32_t w1[15], w2[15];
#pragma unroll
      for (int s = 0, i = 0; s < 4; s++)
#pragma unroll
        for (int gg = 0; gg < (1 << s); gg++, i++) {
          w1[i] = tw[(256 << s) + (row << s) + gg];
          w2[i] = tw[(4096 << s) + (row << (4 + s)) + (c << s) + gg];
        }
      const uint32_t *src = a.modup + g * a.group_stride + loff;
      T x[16];
#pragma unroll
      for (int k = 0; k < 16; k++)
        x[k] = static_cast<T>(ld_at<uint32_t>(src, rbase + (c + 16 * k) * 4u));
#pragma unroll
      for (int s = 0, i = 0; s < 4; s++) {
        const int h = 8 >> s;
#pragma unroll
        for (int gg = 0; gg < (1 << s); gg++, i++) {
          const uint32_t w = w1[i];  // per lane
#pragma unroll
          for (int k = gg * 2 * h; k < gg * 2 * h + h; k++)
            ar.ctv(x[k], x[k + h], w);
        }
      }
#pragma unroll
      for (int k = 0; k < 16; k++) xr[pidx(c + 16 * k)] = x[k];
      wave_lds_sync();
#pragma unroll
      for (int k = 0; k < 16; k++) x[k] = xr[pidx(16 * c + k)];
      wave_lds_sync();
#pragma unroll
      for (int s = 0, i = 0; s < 4; s++) {
        const int h = 8 >> s;
#pragma unroll
        for (int gg = 0; gg < (1 << s); gg++, i++) {
          const uint32_t w = w2[i];  // per lane
#pragma unroll
          for (int k = gg * 2 * h; k < gg * 2 * h + h; k++)
            ar.ctv(x[k], x[k + h], w);
        }
      }
      // columns 16c + k -> the product ownership 4c + 64v + j
#pragma unroll
      for (int k = 0; k < 16; k++) xr[pidx(16 * c + k)] = x[k];
      wave_lds_sync();
#pragma unroll
      for (int k = 0; k < 16; k++)
        u[k] = ar.canon_fwd(xr[pidx(4 * c + 64 * (k >> 2) + (k & 3))]);
      wave_lds_sync();
    }
    const uint32_t *kbp = a.kb[g] + koff;
    const uint32_t *kap = a.ka[g] + koff;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      uint4 tb = ld_at<uint4>(kbp, obase + 256u * v);
      uint4 ta = ld_at<uint4>(kap, obase + 256u * v);
      const uint32_t kbv[4] = {tb.x, tb.y, tb.z, tb.w};
      const uint32_t kav[4] = {ta.x, ta.y, ta.z, ta.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint64_t uv = u[4 * v + j];
        sb[4 * v + j] += uv * kbv[j];
        sa[4 * v + j] += uv * kav[j];
      }
    }
  }
  if (!aux && a.a1 == nullptr && a.cb != nullptr) {
    // CAccum (Context.cpp:684-699): acc += p_prod * ct (bx, and ax if given)
    if (nprod + 1 > 4) fold();
    nprod += 1;
    const uint64_t pp = a.p_prod[l];
    // every load of both polynomials is issued before the first product
    // (a guarded load inside the product loop waited for each in turn)
    const bool with_a = a.ca != nullptr;
    uint4 tb[4], ta[4];
#pragma unroll
    for (int v = 0; v < 4; v++) tb[v] = ld_at<uint4>(a.cb + loff, obase + 256u * v);
    if (with_a) {
#pragma unroll
      for (int v = 0; v < 4; v++) ta[v] = ld_at<uint4>(a.ca + loff, obase + 256u * v);
    }
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const uint32_t cbv[4] = {tb[v].x, tb[v].y, tb[v].z, tb[v].w};
#pragma unroll
      for (int j = 0; j < 4; j++) sb[4 * v + j] += pp * cbv[j];
    }
    if (with_a) {
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const uint32_t cav[4] = {ta[v].x, ta[v].y, ta[v].z, ta[v].w};
#pragma unroll
        for (int j = 0; j < 4; j++) sa[4 * v + j] += pp * cav[j];
      }
    }
  }
  fold();
  if (a.add_b != nullptr) {
    // extended-basis b of a giant-step accumulator, added on every limb
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const uint4 t = ld_at<uint4>(a.add_b + loff, obase + 256u * v);
      const uint32_t tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int j = 0; j < 4; j++) accb[4 * v + j] = add_mod(accb[4 * v + j], tv[j], q);
    }
  }
  (void)qs;
  if (intt_here) {
    // first pass of ModDown's INTT (INTTForModDown, NTT.cu:973-1128) on
    // this limb of both accumulators, straight from the registers; the
    // accumulator itself is not stored
    const uint32_t (&w1)[15] = iw1;
    const uint32_t (&w2)[15] = iw2;
    const size_t ioff = static_cast<size_t>(l - a.intt_lo) << kLogN;
    // back to columns 16c + k, the row pass's input ownership (the group
    // row passes' LDS accesses were this wave's own)
    auto to_rows = [&](uint32_t(&acc)[16]) {
#pragma unroll
      for (int k = 0; k < 16; k++)
        xr[pidx(4 * c + 64 * (k >> 2) + (k & 3))] = acc[k];
      wave_lds_sync();
#pragma unroll
      for (int k = 0; k < 16; k++) acc[k] = xr[pidx(16 * c + k)];
    };
    to_rows(accb);
    inv_rows_body<kLazy>(w1, w2, accb, q, qinv, a.intt_b + ioff, xch);
    __syncthreads();  // the first polynomial's store reads cross rows
    to_rows(acca);
    inv_rows_body<kLazy>(w1, w2, acca, q, qinv, a.intt_a + ioff, xch);
    return;
  }
  uint32_t *ob = a.acc_b + loff;
  uint32_t *oa = a.acc_a + loff;
#pragma unroll
  for (int v = 0; v < 4; v++) {
    st_at<uint4>(ob, obase + 256u * v,
                 make_uint4(accb[4 * v], accb[4 * v + 1], accb[4 * v + 2],
                            accb[4 * v + 3]));
    st_at<uint4>(oa, obase + 256u * v,
                 make_uint4(acca[4 * v], acca[4 * v + 1], acca[4 * v + 2],
                            acca[4 * v + 3]));
  }
}

// grid (kRows / kTileRows, num_q + alpha, jobs)
__global__ __launch_bounds__(256) void modup_keyacc(KeyAccBatch b) {
  __shared__ int32_t xch[kTileRows * kRowPad];
  const chd_keyacc_args &a = b.job[blockIdx.z];
  // limbs in reverse: the aux limbs, which carry a row pass per group and
  // the INTT row passes, are dispatched first and do not form the tail
  const int l = static_cast<int>(gridDim.y - 1 - blockIdx.y);
  const bool aux = l >= a.num_q;
  const int ti = a.tab_off + l + (aux ? a.tab_gap : 0);
  const uint32_t q = b.tab.q[ti];
  const uint32_t qinv = static_cast<uint32_t>(b.tab.qinv[ti]);
  if (q < (1u << 30))
    keyacc_body<true>(a, b.tab, l, aux, ti, q, qinv, xch);
  else
    keyacc_body<false>(a, b.tab, l, aux, ti, q, qinv, xch);
}

// ------------------------------------------------------------------------
// Single-pass forward NTT (out of place): four workgroups per limb, each
// producing one output quarter (index bits 15..14 = j) from one HBM read of
// the limb and one HBM write of its quarter; the intermediate never leaves
// the CU. Stages 0 and 1 are the only ones that mix quarters: a workgroup
// recomputes just the one of their four outputs that lies in its quarter,
//   z_j[n'] = x0 + s1 w1 x1 + s0 w0 x2 + s0 s1 w0 w1 x3,   x_m = x[n' + 2^14 m]
// (w0 = psi_rev[1], w1 = psi_rev[2 + (j >> 1)], s0 = -1 for j >= 2, s1 = -1
// for odd j), the same residue the reference's first two butterfly stages
// give (NTT.cu:231-338). Stages 2..15 then run in four register rounds of
// the bits 13..10 | 9..6 | 5..2 | 1..0 with three LDS exchanges; the last
// round owns 4 consecutive outputs per lane, so every wave stores 1 KiB
// contiguous per instruction.
// The four workgroups of a limb get block ids 8 apart (the same XCD under
// round-robin dispatch) so three of the four reads of the limb hit in L2.
// ------------------------------------------------------------------------
// Opt-in instrumentation (built only with CHD_PHASE_TIMESTAMPS, never in
// the product library): each wave of ntt_fwd_1p writes the 100 MHz
// real-time clock at its phase boundaries (start, round-1 loads done, round 1
// done, barrier passed, round 2 done, round 3 done, stores done) into a
// buffer of 8 words per wave, lane 0 with an ordinary vector store.
#ifdef CHD_PHASE_TIMESTAMPS
__device__ unsigned long long *g_phase_ts = nullptr;
__device__ int g_phase_waves = 0;
__device__ __forceinline__ void phase_mark(int slot) {
  const int wid = blockIdx.x * 16 + (threadIdx.x >> 6);
  const unsigned long long now = __builtin_amdgcn_s_memrealtime();
  if ((threadIdx.x & 63) == 0 && g_phase_ts != nullptr &&
      wid < g_phase_waves && slot >= 0 && slot < 8)
    g_phase_ts[wid * 8 + slot] = now;
}
#define CHD_PHASE(k) phase_mark(k)
#else
#define CHD_PHASE(k)
#endif

constexpr int kQuarter = kN / 4;
constexpr int kQLdsWords = kQuarter + kQuarter / 16;  // 4 pad words per 64
__device__ __forceinline__ int qidx(int n) { return n + ((n >> 6) << 2); }


// radix-16 over the 16 registers; stage t (0..3) has 2^t groups and group g
// uses tw[base[t] + g]; kUniform: the twiddles are wave-uniform; kRed0
// false: the inputs lie in [0, 2q), so stage 0 needs no reduction
template <bool kUniform, bool kRed0, typename A>
__device__ __forceinline__ void radix16_1p(const A &ar,
                                           typename A::T (&x)[16],
                                           const uint32_t *tw,
                                           const int (&base)[4]) {
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int h = 8 >> t;
#pragma unroll
    for (int g = 0; g < (1 << t); g++) {
      const uint32_t w = kUniform ? ld_uniform(tw, base[t] + g) : tw[base[t] + g];
      const uint32_t wq = ar.twq(w);
#pragma unroll
      for (int k = g * 2 * h; k < g * 2 * h + h; k++) {
        if (t == 0 && !kRed0)
          ar.template ct<false>(x[k], x[k + h], w, wq);
        else
          ar.ct(x[k], x[k + h], w, wq);
      }
    }
  }
}

// radix-16 with the 15 twiddles of its four stages preloaded:
// w[(1 << t) - 1 + g] is group g of stage t. kVec: the twiddles are per lane
// (no companion multiply); otherwise wave-uniform (scalar companion).
template <bool kVec, typename A>
__device__ __forceinline__ void radix16_pre(const A &ar,
                                            typename A::T (&x)[16],
                                            const uint32_t (&w)[15]) {
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int h = 8 >> t;
#pragma unroll
    for (int g = 0; g < (1 << t); g++) {
      const uint32_t wv = w[(1 << t) - 1 + g];
      if constexpr (kVec) {
#pragma unroll
        for (int k = g * 2 * h; k < g * 2 * h + h; k++)
          ar.ctv(x[k], x[k + h], wv);
      } else {
        const uint32_t wq = ar.twq(wv);
#pragma unroll
        for (int k = g * 2 * h; k < g * 2 * h + h; k++)
          ar.ct(x[k], x[k + h], wv, wq);
      }
    }
  }
}

// kPre: the input times a per-limb MontMul constant cst[l] on the way in.
// With the store epilogue that is the Montgomery conversion; with the ModDown
// epilogue the source is broadcast: every limb of polynomial z transforms the
// same centred (signed) limb src + z * src_pstride times its cst[l], i.e. the
// output of a one-source BConv (ModSwitch.cu:23-171 with one source:
// y_l = c T_l 2^-32 mod q_l) that is never stored.
// round-1 input word: streaming for a limb's own input (its four
// workgroups read it together), default caching for a broadcast source,
// which every workgroup of the polynomial reads and the L2 keeps for them
template <int kEpi, bool kPre, bool kLazy>
__device__ __forceinline__ void fwd_1p_body(const NttArgs &a, const Limb &lb,
                                            int z, int j, uint32_t q,
                                            uint32_t qinv, uint32_t *lds) {
  using A = Arith<kLazy>;
  using T = typename A::T;
  constexpr bool kBcast = kPre && kEpi == kEpiModDown;
  // round-1 input words: streaming for a limb's own input (its four
  // workgroups read it together), default caching for a broadcast source,
  // which every workgroup of the polynomial reads and the L2 keeps for them
  constexpr int kSrcAux = kBcast ? 0 : 2;
  const A ar(q, qinv);
  const uint32_t *tw = a.tab.tw + (static_cast<size_t>(lb.ti) << kLogN);
  const uint32_t *src =
      a.src + z * a.src_pstride +
      (kBcast ? size_t{0} : static_cast<size_t>(lb.sl) << kLogN);
  uint32_t *dst = poly_dst(a, z) + (static_cast<size_t>(lb.l) << kLogN) +
                  j * kQuarter;
  const rsrc_t rtw = make_rsrc(tw, 4u * kN);
  const rsrc_t rsrc = make_rsrc(src, 4u * kN);
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  CHD_PHASE(0);
  // Twiddles of rounds 2-4, requested before the round-1 loads: after the
  // workgroup barrier every wave of the CU computes at once, and a round
  // that first waited for its twiddles would leave the VALUs idle
  // (round 2: wave-uniform, w[(1 << s) - 1 + g] = psi_rev[((64 + hi) << s)
  // + g]; round 3: per lane, the same from 1024, the 2^s words of stage s
  // contiguous and 2^s-aligned, so one or two vector loads each; round 4:
  // per store round v, psi_rev[16384 + hi4] and the pair at
  // psi_rev[32768 + 2 hi4]). Per-lane offsets in the VGPR operand, the
  // wave-uniform rest in the scalar one.
  uint32_t w2[15], w3[15], w4[4][3];
  {
    const int hi2 = (j << 4) | wave;              // bits 15..10
    const uint32_t u3 = 1024u + ((j << 8) | (wave << 4));  // + (lane >> 2)
    const uint32_t l3 = static_cast<uint32_t>(lane >> 2);
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
      for (int g = 0; g < (1 << s); g++)
        w2[(1 << s) - 1 + g] = ld_uniform(tw, ((64 + hi2) << s) + g);
    w3[0] = bld1(rtw, l3 << 2, u3 << 2);
    const u32x2 p1 = bld2(rtw, l3 << 3, u3 << 3);
    w3[1] = p1[0];
    w3[2] = p1[1];
    const u32x4 p2 = bld4(rtw, l3 << 4, u3 << 4);
#pragma unroll
    for (int i = 0; i < 4; i++) w3[3 + i] = p2[i];
    const u32x4 p3a = bld4(rtw, l3 << 5, u3 << 5);
    const u32x4 p3b = bld4(rtw, (l3 << 5) + 16u, u3 << 5);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      w3[7 + i] = p3a[i];
      w3[11 + i] = p3b[i];
    }
#pragma unroll
    for (int v = 0; v < 4; v++) {
      // hi4 = (j << 12) | (wave << 8) | (v << 6) | lane: bits 15..2
      const uint32_t u4 =
          static_cast<uint32_t>((j << 12) | (wave << 8) | (v << 6));
      w4[v][0] = bld1(rtw, static_cast<uint32_t>(lane) << 2,
                      (16384u + u4) << 2);
      const u32x2 pb = bld2(rtw, static_cast<uint32_t>(lane) << 3,
                            (32768u + 2u * u4) << 2);
      w4[v][1] = pb[0];
      w4[v][2] = pb[1];
    }
  }
  const uint32_t w0 = ld_uniform(tw, 1);
  const uint32_t w1 = ld_uniform(tw, 2 + (j >> 1));
  // lane part of every round-1 input offset; quarter m and row k of the
  // lane's 16 go in the scalar offset
  const uint32_t vt = 4u * static_cast<uint32_t>(t);
  T x[16];
  // ---- round 1: stages 0, 1 of quarter j (bits 15, 14), then 2..5
  if constexpr (kLazy) {
    // one 64-bit dot product and one reduction per output: with canonical
    // inputs and constants below q < 2^30 the sum stays below q 2^32
    const uint32_t qn = ar.qn;
    const uint32_t w01 = mont_mad(w0, w1, w1 * qn, q);
    uint32_t c[4];
    c[0] = ld_uniform(tw, 0);  // ToMont(1)
    c[1] = (j & 1) ? q - w1 : w1;
    c[2] = (j >> 1) ? q - w0 : w0;
    const uint32_t w01c = umin(w01, w01 - q);
    c[3] = (((j >> 1) ^ j) & 1) ? q - w01c : w01c;
    if constexpr (kPre) {
      // the prologue constant (Montgomery conversion, or the one-source
      // BConv table entry of this limb) folded into the constants
      const uint32_t ce = a.cst[lb.ci];
      const uint32_t cen = ce * qn;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t v = mont_mad(c[i], ce, cen, q);
        c[i] = umin(v, v - q);
      }
    }
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const uint32_t so = 4u * static_cast<uint32_t>(k << 10);
      const uint32_t x0 = bld1<kSrcAux>(rsrc, vt, so);
      const uint32_t x1 = bld1<kSrcAux>(rsrc, vt, so + 4u * kQuarter);
      const uint32_t x2 = bld1<kSrcAux>(rsrc, vt, so + 8u * kQuarter);
      const uint32_t x3 = bld1<kSrcAux>(rsrc, vt, so + 12u * kQuarter);
      uint64_t acc;
      if constexpr (kBcast) {
        // centred inputs of a source prime below 2^31, |x| < 2^30, times
        // constants below q: the signed sum lies in (-q 2^32, q 2^32);
        // adding q 2^32 (= 0 mod q) makes it positive and below q 2^33 <
        // 2^63, and the reduction below then lands in [0, 3q), inside the
        // [0, 4q) the butterflies take
        acc = static_cast<uint64_t>(
            (static_cast<int64_t>(q) << 32) +
            static_cast<int64_t>(static_cast<int32_t>(x0)) *
                static_cast<int32_t>(c[0]) +
            static_cast<int64_t>(static_cast<int32_t>(x1)) *
                static_cast<int32_t>(c[1]) +
            static_cast<int64_t>(static_cast<int32_t>(x2)) *
                static_cast<int32_t>(c[2]) +
            static_cast<int64_t>(static_cast<int32_t>(x3)) *
                static_cast<int32_t>(c[3]));
      } else {
        acc = static_cast<uint64_t>(x0) * c[0] +
              static_cast<uint64_t>(x1) * c[1] +
              static_cast<uint64_t>(x2) * c[2] +
              static_cast<uint64_t>(x3) * c[3];
      }
      const uint32_t m = static_cast<uint32_t>(acc) * qn;
      x[k] = static_cast<uint32_t>((static_cast<uint64_t>(m) * q + acc) >> 32);
    }
  } else {
    // reference-form butterflies, keeping the half of each that lies in
    // quarter j (NTTUtils.cuh:19-34)
    const int32_t qs = static_cast<int32_t>(q);
    const int32_t w0s = static_cast<int32_t>(w0);
    const int32_t w0q = static_cast<int32_t>(w0 * qinv);
    const int32_t w1s = static_cast<int32_t>(w1);
    const int32_t w1q = static_cast<int32_t>(w1 * qinv);
    int32_t ce = 0, ceq = 0;
    if constexpr (kPre) {
      ce = static_cast<int32_t>(a.cst[lb.ci]);
      ceq = static_cast<int32_t>(static_cast<uint32_t>(ce) * qinv);
    }
    const bool hi0 = j >= 2, hi1 = j & 1;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const uint32_t so = 4u * static_cast<uint32_t>(k << 10);
      int32_t xm[4];
#pragma unroll
      for (int m = 0; m < 4; m++) {
        xm[m] = static_cast<int32_t>(
            bld1<kSrcAux>(rsrc, vt, so + 4u * kQuarter * m));
        // (a broadcast source is centred: mont takes signed inputs)
        if constexpr (kPre) xm[m] = mont(xm[m], ce, ceq, qs);
      }
      ct_bfly(xm[0], xm[2], w0s, w0q, qs);
      ct_bfly(xm[1], xm[3], w0s, w0q, qs);
      int32_t ya = hi0 ? xm[2] : xm[0];
      int32_t yb = hi0 ? xm[3] : xm[1];
      ct_bfly(ya, yb, w1s, w1q, qs);
      x[k] = hi1 ? yb : ya;
    }
  }
  CHD_PHASE(1);
  {
    // the lazy prologue's outputs lie in [0, 2q) (dot product of canonical
    // values below q 2^32 reduced), except for the broadcast form's [0, 3q)
    const int base[4] = {4 + j, 8 + 2 * j, 16 + 4 * j, 32 + 8 * j};
    radix16_1p<true, kBcast>(ar, x, tw, base);
  }
  CHD_PHASE(2);
  T *xs = reinterpret_cast<T *>(lds);
#pragma unroll
  for (int k = 0; k < 16; k++) xs[qidx((k << 10) | t)] = x[k];
  __syncthreads();
  CHD_PHASE(3);
  // From here on each wave reads and writes only its own 1024-element block
  // (index bits 13..10 = wave), so the exchanges of rounds 3 and 4 need no
  // workgroup barrier.
  // ---- round 2: stages 6..9 (bits 9..6); lane = bits 5..0, wave = 13..10
#pragma unroll
  for (int k = 0; k < 16; k++) x[k] = xs[qidx((wave << 10) | (k << 6) | lane)];
  radix16_pre<false>(ar, x, w2);
#pragma unroll
  for (int k = 0; k < 16; k++) xs[qidx((wave << 10) | (k << 6) | lane)] = x[k];
  wave_lds_sync();
  CHD_PHASE(4);
  // ---- round 3: stages 10..13 (bits 5..2); lane = bits 9..6 | bits 1..0
  const int b96 = lane >> 2, b10 = lane & 3;
#pragma unroll
  for (int k = 0; k < 16; k++)
    x[k] = xs[qidx((wave << 10) | (b96 << 6) | (k << 2) | b10)];
  radix16_pre<true>(ar, x, w3);
#pragma unroll
  for (int k = 0; k < 16; k++)
    xs[qidx((wave << 10) | (b96 << 6) | (k << 2) | b10)] = x[k];
  wave_lds_sync();
  CHD_PHASE(5);
  // ---- round 4: stages 14, 15 (bits 1..0); lane = bits 7..2, wave =
  // bits 13..10, store round v = bits 9..8
  const int32_t qs = static_cast<int32_t>(q);
  [[maybe_unused]] int32_t c2 = 0, c2q = 0, pe = 0, peq = 0;
  [[maybe_unused]] bool has_pad = false;
  [[maybe_unused]] bool has_s2 = false;
  [[maybe_unused]] rsrc_t rs2 = make_rsrc(src, 0);
  if constexpr (kEpi == kEpiModDown) {
    c2 = static_cast<int32_t>(a.cst2[lb.l]);
    c2q = static_cast<int32_t>(static_cast<uint32_t>(c2) * qinv);
    if (lb.l >= a.src2_lo && lb.l < a.src2_hi) {
      has_s2 = true;
      rs2 = make_rsrc(a.src2 + z * a.src2_pstride +
                          (static_cast<size_t>(lb.l - a.src2_lo) << kLogN) +
                          j * kQuarter,
                      4u * kQuarter);
      if (a.pad != nullptr) {
        has_pad = true;
        pe = static_cast<int32_t>(a.pad[lb.l - a.src2_lo]);
        peq = static_cast<int32_t>(static_cast<uint32_t>(pe) * qinv);
      }
    }
  }
  const uint32_t vl = static_cast<uint32_t>(lane) << 4;
  // the epilogue's src2 words of all four store rounds, requested together
  // (one guarded load per round waited for each in turn)
  [[maybe_unused]] u32x4 s2v[4];
  if constexpr (kEpi == kEpiModDown) {
#pragma unroll
    for (int v = 0; v < 4; v++) s2v[v] = u32x4{0, 0, 0, 0};
    if (has_s2) {
#pragma unroll
      for (int v = 0; v < 4; v++)
        s2v[v] = bld4<2>(rs2, vl,
                         4u * static_cast<uint32_t>((wave << 10) | (v << 8)));
    }
  }
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int n = (wave << 10) | (v << 8) | (lane << 2);
    const uint32_t sn = 4u * static_cast<uint32_t>((wave << 10) | (v << 8));
    [[maybe_unused]] u32x4 s2 = {0, 0, 0, 0};
    if constexpr (kEpi == kEpiModDown) s2 = s2v[v];
    const u32x4 u = *reinterpret_cast<const u32x4 *>(&lds[qidx(n)]);
    T y[4];
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] = static_cast<T>(u[i]);
    const uint32_t wa = w4[v][0];
    ar.ctv(y[0], y[2], wa);
    ar.ctv(y[1], y[3], wa);
    ar.ctv(y[0], y[1], w4[v][1]);
    ar.ctv(y[2], y[3], w4[v][2]);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = ar.canon_fwd(y[i]);
    if constexpr (kEpi == kEpiModDown) {
      // NTTPhase2ForModDown epilogue (NTT.cu:567-600):
      // MontMul(MontMul(src2, pad) - y, inv_prod), zero src2 outside
      // [src2_lo, src2_hi)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        int32_t sv = static_cast<int32_t>(s2[i]);
        if (has_pad) sv = norm(mont(sv, pe, peq, qs), qs);
        const int32_t dv = sv - static_cast<int32_t>(o[i]);
        o[i] = static_cast<uint32_t>(norm(mont(dv, c2, c2q, qs), qs));
      }
    }
    // the wave-uniform part of the address in the scalar base
    st_nt<u32x4>(dst + (sn >> 2), vl, o);
  }
  CHD_PHASE(6);
}

// grid: 1D, 4 * roundup(limbs * polys, 8) blocks of 1024 threads
template <int kEpi, bool kPre>
__device__ __forceinline__ void fwd_1p_entry(const NttArgs &a, int num_limbs,
                                             int num_items, uint32_t *lds) {
  const int b = blockIdx.x;
  const int slot = b >> 3;
  const int j = slot & 3;
  const int li = (slot >> 2) * 8 + (b & 7);
  if (li >= num_items) return;
  const int z = li / num_limbs;
  const Limb lb = decode(a.map, li - z * num_limbs);
  const uint32_t q = a.tab.q[lb.ti];
  const uint32_t qinv = static_cast<uint32_t>(a.tab.qinv[lb.ti]);
  if (q < (1u << 30))
    fwd_1p_body<kEpi, kPre, true>(a, lb, z, j, q, qinv, lds);
  else
    fwd_1p_body<kEpi, kPre, false>(a, lb, z, j, q, qinv, lds);
}

// At most 64 VGPRs (8 waves per SIMD): two of these workgroups (16 waves,
// 68 KiB of LDS each) fit on one CU, so a launch on another stream can run
// its loads beside this one's butterflies. The broadcast ModDown form needs
// more registers and keeps the default limit (ntt_fwd_1p_bcast), and so does
// the phase-timestamp build, whose marks would otherwise spill.
#ifdef CHD_PHASE_TIMESTAMPS
#define CHD_FWD_1P_WAVES
#else
#define CHD_FWD_1P_WAVES __attribute__((amdgpu_waves_per_eu(8)))
#endif
template <int kEpi, bool kPre>
__global__ __launch_bounds__(1024) CHD_FWD_1P_WAVES
void ntt_fwd_1p(NttArgs a, int num_limbs, int num_items) {
  __shared__ __align__(16) uint32_t lds[kQLdsWords];
  fwd_1p_entry<kEpi, kPre>(a, num_limbs, num_items, lds);
}

__global__ __launch_bounds__(1024) void ntt_fwd_1p_bcast(NttArgs a,
                                                         int num_limbs,
                                                         int num_items) {
  __shared__ __align__(16) uint32_t lds[kQLdsWords];
  fwd_1p_entry<kEpiModDown, true>(a, num_limbs, num_items, lds);
}

// ------------------------------------------------------------------------
// Single-pass inverse over residue classes of the output.
// With input index i = 4k + r (r < 4, k < N/4), brev(i) = brev2(r) 2^14 +
// brev14(k), so the kernels' N intt (INTT of NTT.cu:23-229 without N^-1) is
//   S[4u + s] = sum_k psi^-(e_k (4u + s)) D_s[k],   e_k = 2 brev14(k) + 1,
//   D_s[k]    = sum_r y[4k + r] I^-(brev2(r) s),    I = psi^(N/2)
//             = sum_k (psi^4)^-(e_k u) Z_s[k],      Z_s[k] = psi^-(s e_k) D_s[k]:
// for each residue class s of the output, the N/4-point inverse with root
// psi^4, whose twiddles (psi^4)^-brev14(m) are psi_inv_rev[m] for m < N/4,
// of the four adjacent input words combined with constants and twisted.
// Workgroup s of a limb computes class s: it reads the whole limb (16-byte
// loads of y[4k .. 4k + 3]) and writes every fourth word of it. The
// epilogue constant is folded into the four combination constants, so the
// last round only makes the values canonical (or centred).
// The four register rounds mirror the forward single pass's, in reverse:
// stage bits 1..0 and 5..2 (per-lane twiddles), 9..6 (wave-uniform) and
// 13..10 (uniform), through the same LDS layouts; only the last exchange
// crosses waves.
// ------------------------------------------------------------------------

// GS radix-16 over the 16 registers: stage t (0..3) pairs registers j and
// j + 2^t (bit t of j clear); group gg = j >> (t + 1) of stage t uses
// w[16 - (16 >> t) + gg]. kVec: per-lane twiddles (no companion multiply).
template <bool kVec, typename A>
__device__ __forceinline__ void radix16_gs(const A &ar,
                                           typename A::T (&x)[16],
                                           const uint32_t (&w)[15]) {
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int h = 1 << t;
#pragma unroll
    for (int gg = 0; gg < (8 >> t); gg++) {
      const uint32_t wv = w[16 - (16 >> t) + gg];
      if constexpr (kVec) {
#pragma unroll
        for (int p = 0; p < h; p++)
          ar.gsv(x[gg * 2 * h + p], x[gg * 2 * h + p + h], wv);
      } else {
        const uint32_t wq = ar.twq(wv);
#pragma unroll
        for (int p = 0; p < h; p++)
          ar.gs(x[gg * 2 * h + p], x[gg * 2 * h + p + h], wv, wq);
      }
    }
  }
}

template <int kEpi, bool kLazy>
__device__ __forceinline__ void inv_1p_body(const NttArgs &a, const Limb &lb,
                                            int z, int s, uint32_t q,
                                            uint32_t qinv, uint32_t *lds) {
  using A = Arith<kLazy>;
  using T = typename A::T;
  const A ar(q, qinv);
  const uint32_t *itw = a.tab.itw + (static_cast<size_t>(lb.ti) << kLogN);
  const uint32_t *src = a.src + z * a.src_pstride +
                        (static_cast<size_t>(lb.sl) << kLogN);
  // output class s: word 4u + s of the limb
  uint32_t *dst = poly_dst(a, z) + (static_cast<size_t>(lb.l) << kLogN) + s;
  const rsrc_t ritw = make_rsrc(itw, 4u * kN);
  const rsrc_t rsrc = make_rsrc(src, 4u * kN);
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int32_t qs = static_cast<int32_t>(q);
  const uint32_t qn = 0u - qinv;
  // Per-lane twiddles of rounds 1 and 2 and the twists, requested before
  // the input (round 1, store round v: hi4 = k >> 2 = (wave << 8) |
  // (v << 6) | lane, psi_inv_rev[8192 + 2 hi4 + {0, 1}] and [4096 + hi4];
  // round 2: hi = k >> 6 = (wave << 4) | (lane >> 2), stage t's 8 >> t
  // words at psi_inv_rev[2^(11 - t) + (hi << (3 - t))]).
  uint32_t w1[4][3], w2[15];
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const uint32_t u4 = static_cast<uint32_t>((wave << 8) | (v << 6));
    const u32x2 pb = bld2(ritw, static_cast<uint32_t>(lane) << 3,
                          (8192u + 2u * u4) << 2);
    w1[v][0] = pb[0];
    w1[v][1] = pb[1];
    w1[v][2] = bld1(ritw, static_cast<uint32_t>(lane) << 2, (4096u + u4) << 2);
  }
  {
    const uint32_t b96 = static_cast<uint32_t>(lane >> 2);
    const uint32_t u2 = static_cast<uint32_t>(wave << 4);
    const u32x4 pa = bld4(ritw, b96 << 5, (2048u + 8u * u2) << 2);
    const u32x4 pb = bld4(ritw, (b96 << 5) + 16u, (2048u + 8u * u2) << 2);
    const u32x4 pc = bld4(ritw, b96 << 4, (1024u + 4u * u2) << 2);
    const u32x2 pd = bld2(ritw, b96 << 3, (512u + 2u * u2) << 2);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      w2[i] = pa[i];
      w2[4 + i] = pb[i];
      w2[8 + i] = pc[i];
    }
    w2[12] = pd[0];
    w2[13] = pd[1];
    w2[14] = bld1(ritw, b96 << 2, (256u + u2) << 2);
  }
  // round-1 input layout (the forward's round-2 layout): register rho =
  // k bits 9..6, lane = bits 5..0, wave = bits 13..10; element k reads the
  // 16 bytes y[4k .. 4k + 3]
  // twists of this class (ToMont(1) for class 0: no branch in the loop
  // below, whose loads then stay in flight together)
  uint32_t tau[16];
  {
    const rsrc_t rtau = make_rsrc(
        a.tab.twist + (static_cast<size_t>(lb.ti) * 4 + s) * kQuarter,
        4u * kQuarter);
#pragma unroll
    for (int rho = 0; rho < 16; rho++)
      tau[rho] = bld1(rtau, static_cast<uint32_t>(lane) << 2,
                      4u * static_cast<uint32_t>((wave << 10) | (rho << 6)));
  }
  // combination constants c_r = I^-(brev2(r) s) times the epilogue
  // constant, canonical: I^-e for e = 0..3 is ToMont(1), psi_inv_rev[1],
  // -ToMont(1), -psi_inv_rev[1]
  uint32_t cc[4];
  {
    const uint32_t one = ld_uniform(itw, 0), ii = ld_uniform(itw, 1);
    const uint32_t ce = a.cst[lb.ci];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int br = ((r & 1) << 1) | (r >> 1);
      const int e = (br * s) & 3;
      const uint32_t c = e == 0 ? one : e == 1 ? ii : e == 2 ? q - one : q - ii;
      const uint32_t v = mont_mad(c, ce, ce * qn, q);  // [0, 2q) for q < 2^31
      cc[r] = v >= q ? v - q : v;
    }
  }
  T x[16];
#pragma unroll
  for (int rho = 0; rho < 16; rho++) {
    const u32x4 y = bld4<2>(rsrc, static_cast<uint32_t>(lane) << 4,
                            16u * static_cast<uint32_t>((wave << 10) |
                                                        (rho << 6)));
    if constexpr (kLazy) {
      // inputs below 2q: the sum is below 8 q^2, its reduction below 3q, and
      // the twist's product reduces into [0, 2q)
      const uint64_t acc = static_cast<uint64_t>(y[0]) * cc[0] +
                           static_cast<uint64_t>(y[1]) * cc[1] +
                           static_cast<uint64_t>(y[2]) * cc[2] +
                           static_cast<uint64_t>(y[3]) * cc[3];
      const uint32_t m = static_cast<uint32_t>(acc) * qn;
      uint32_t d =
          static_cast<uint32_t>((static_cast<uint64_t>(m) * q + acc) >> 32);
      x[rho] = mont_lo(d, tau[rho], qn, q);  // [0, 2q)
    } else {
      // reference form: canonical inputs (signed ones in (-q, q) as well)
      uint64_t acc = 0;
#pragma unroll
      for (int i = 0; i < 4; i++)
        acc += static_cast<uint64_t>(
                   static_cast<uint32_t>(norm(static_cast<int32_t>(y[i]), qs))) *
               cc[i];
      const int32_t d = static_cast<int32_t>(reduce_sum4(acc, q, qn));
      x[rho] = mont_s(d, static_cast<int32_t>(tau[rho]), qinv, qs);  // (-q, q)
    }
  }
  T *xs = reinterpret_cast<T *>(lds);
#pragma unroll
  for (int rho = 0; rho < 16; rho++)
    xs[qidx((wave << 10) | (rho << 6) | lane)] = x[rho];
  wave_lds_sync();
  // ---- round 1: stages on bits 1..0 (the forward's round-4 layout: lane =
  // bits 7..2, store round v = bits 9..8, the four words of a lane = bits
  // 1..0)
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int n = (wave << 10) | (v << 8) | (lane << 2);
    u32x4 u = *reinterpret_cast<const u32x4 *>(&lds[qidx(n)]);
    T y[4];
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] = static_cast<T>(u[i]);
    ar.gsv(y[0], y[1], w1[v][0]);
    ar.gsv(y[2], y[3], w1[v][1]);
    ar.gsv(y[0], y[2], w1[v][2]);
    ar.gsv(y[1], y[3], w1[v][2]);
#pragma unroll
    for (int i = 0; i < 4; i++) u[i] = static_cast<uint32_t>(y[i]);
    *reinterpret_cast<u32x4 *>(&lds[qidx(n)]) = u;
  }
  wave_lds_sync();
  // ---- round 2: stages on bits 5..2 (the forward's round-3 layout)
  {
    const int b96 = lane >> 2, b10 = lane & 3;
#pragma unroll
    for (int rho = 0; rho < 16; rho++)
      x[rho] = xs[qidx((wave << 10) | (b96 << 6) | (rho << 2) | b10)];
    radix16_gs<true>(ar, x, w2);
#pragma unroll
    for (int rho = 0; rho < 16; rho++)
      xs[qidx((wave << 10) | (b96 << 6) | (rho << 2) | b10)] = x[rho];
  }
  wave_lds_sync();
  // ---- round 3: stages on bits 9..6 (the forward's round-2 layout);
  // twiddles wave-uniform: psi_inv_rev[2^(7 - t) + (wave << (3 - t)) + gg]
  {
    uint32_t w3[15];
#pragma unroll
    for (int tt = 0; tt < 4; tt++)
#pragma unroll
      for (int gg = 0; gg < (8 >> tt); gg++)
        w3[16 - (16 >> tt) + gg] =
            ld_uniform(itw, (128 >> tt) + (wave << (3 - tt)) + gg);
#pragma unroll
    for (int rho = 0; rho < 16; rho++)
      x[rho] = xs[qidx((wave << 10) | (rho << 6) | lane)];
    radix16_gs<false>(ar, x, w3);
#pragma unroll
    for (int rho = 0; rho < 16; rho++)
      xs[qidx((wave << 10) | (rho << 6) | lane)] = x[rho];
  }
  __syncthreads();
  // ---- round 4: stages on bits 13..10 (the forward's round-1 layout: the
  // register is bits 13..10, the thread bits 9..0); twiddles uniform:
  // psi_inv_rev[2^(3 - t) + gg]
  {
    uint32_t w4[15];
#pragma unroll
    for (int tt = 0; tt < 4; tt++)
#pragma unroll
      for (int gg = 0; gg < (8 >> tt); gg++)
        w4[16 - (16 >> tt) + gg] = ld_uniform(itw, (8 >> tt) + gg);
#pragma unroll
    for (int rho = 0; rho < 16; rho++) x[rho] = xs[qidx((rho << 10) | t)];
    radix16_gs<false>(ar, x, w4);
  }
  // output u = (rho << 10) | t is word 4u + s: every fourth word, written
  // with default caching so that the limb's four workgroups (one XCD, one
  // L2) complete each line before it leaves the L2
#pragma unroll
  for (int rho = 0; rho < 16; rho++) {
    int32_t v = static_cast<int32_t>(ar.canon_inv(x[rho]));
    if constexpr (kEpi == kEpiConstCentre)
      if (v > (qs >> 1)) v -= qs;
    st_at<int32_t>(dst + (rho << 12), 16u * static_cast<uint32_t>(t), v);
  }
}

// grid: 1D, 4 * roundup(limbs * polys, 8) blocks of 1024 threads (the four
// classes of a limb 8 block ids apart: one XCD)
template <int kEpi>
__global__ __launch_bounds__(1024) void ntt_inv_1p(NttArgs a, int num_limbs,
                                                   int num_items) {
  __shared__ __align__(16) uint32_t lds[kQLdsWords];
  const int b = blockIdx.x;
  const int slot = b >> 3;
  const int s = slot & 3;
  const int li = (slot >> 2) * 8 + (b & 7);
  if (li >= num_items) return;
  const int z = li / num_limbs;
  const Limb lb = decode(a.map, li - z * num_limbs);
  const uint32_t q = a.tab.q[lb.ti];
  const uint32_t qinv = static_cast<uint32_t>(a.tab.qinv[lb.ti]);
  if (q < (1u << 30))
    inv_1p_body<kEpi, true>(a, lb, z, s, q, qinv, lds);
  else
    inv_1p_body<kEpi, false>(a, lb, z, s, q, qinv, lds);
}

}  // namespace

hipError_t launch_ntt_fwd_cols(const NttArgs &a, int num_limbs, int num_z,
                               hipStream_t s) {
  if (num_limbs <= 0 || num_z <= 0) return hipSuccess;
  dim3 gc(kCols / kTileCols, num_limbs, num_z);
  hipLaunchKernelGGL(ntt_fwd_cols<false>, gc, dim3(512), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_ntt_fwd_rows(const NttArgs &a, int num_limbs, int num_z,
                               hipStream_t s) {
  if (num_limbs <= 0 || num_z <= 0) return hipSuccess;
  dim3 gr(kRows / kTileRows, num_limbs, num_z);
  hipLaunchKernelGGL(ntt_fwd_rows<kEpiStore>, gr, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_modup_keyacc(const KeyAccBatch &a, int num_jobs,
                               hipStream_t s) {
  dim3 g(kRows / kTileRows, a.job[0].num_q + a.job[0].alpha, num_jobs);
  hipLaunchKernelGGL(modup_keyacc, g, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_ntt_fwd(const NttArgs &a, int num_limbs, int num_polys,
                          bool pre_const, int epilogue, hipStream_t s) {
  if (num_limbs <= 0 || num_polys <= 0) return hipSuccess;
  // The single pass takes one workgroup's latency however few limbs there
  // are (12.3 us for 1 limb, 13.9 for 16, 16-17 for 64); up to 16 limbs
  // the two passes, spread over many small workgroups, are faster (9.3 us
  // for 1 limb, 11.3-12.5 for 2-16; from 24 limbs on they are not). The
  // ModDown epilogue keeps the single pass: its caller makes that choice.
  const int items = num_limbs * num_polys;
  if (a.src_disjoint && !a.fwd_two_pass &&
      (epilogue == kEpiModDown || items > 16)) {
    dim3 g1(4 * ((items + 7) / 8 * 8));
    if (epilogue == kEpiModDown && a.src_bcast)
      hipLaunchKernelGGL(ntt_fwd_1p_bcast, g1, dim3(1024), 0, s, a,
                         num_limbs, items);
    else if (epilogue == kEpiModDown)
      hipLaunchKernelGGL((ntt_fwd_1p<kEpiModDown, false>), g1, dim3(1024), 0,
                         s, a, num_limbs, items);
    else if (pre_const)
      hipLaunchKernelGGL((ntt_fwd_1p<kEpiStore, true>), g1, dim3(1024), 0, s,
                         a, num_limbs, items);
    else
      hipLaunchKernelGGL((ntt_fwd_1p<kEpiStore, false>), g1, dim3(1024), 0, s,
                         a, num_limbs, items);
    return hipGetLastError();
  }
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

hipError_t launch_ntt_inv_cols(const NttArgs &a, int num_limbs, int num_polys,
                               int epilogue, hipStream_t s) {
  dim3 gc(kCols / kTileCols, num_limbs, num_polys);
  if (epilogue == kEpiConstCentre)
    hipLaunchKernelGGL(ntt_inv_cols<kEpiConstCentre>, gc, dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL(ntt_inv_cols<kEpiConst>, gc, dim3(512), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_ntt_inv(const NttArgs &a, int num_limbs, int num_polys,
                          int epilogue, hipStream_t s) {
  if (num_limbs <= 0 || num_polys <= 0) return hipSuccess;
  // The single pass over residue classes (one HBM read and write of each
  // limb instead of two: 43 MB against 76 MB at config 2) runs only when
  // asked for (chd_k_ntt_inv_1p): at config 2 it takes 21.5 us against
  // 19 us for the two passes, and the three-stream headline step 30.3 us
  // against 27.7 us (its every-fourth-word stores cost ~3 us).
  const int items = num_limbs * num_polys;
  if (a.inv_one_pass) {
    dim3 g1(4 * ((items + 7) / 8 * 8));
    if (epilogue == kEpiConstCentre)
      hipLaunchKernelGGL(ntt_inv_1p<kEpiConstCentre>, g1, dim3(1024), 0, s, a,
                         num_limbs, items);
    else
      hipLaunchKernelGGL(ntt_inv_1p<kEpiConst>, g1, dim3(1024), 0, s, a,
                         num_limbs, items);
    return hipGetLastError();
  }
  dim3 gr(kRows / kTileRows, num_limbs, num_polys);
  hipLaunchKernelGGL(ntt_inv_rows, gr, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // the column pass works in place on dst
  NttArgs b = a;
  b.map.src_gap = 0;
  return launch_ntt_inv_cols(b, num_limbs, num_polys, epilogue, s);
}

}  // namespace chd

using namespace chd;

namespace {
// limbs one polynomial of a strided operand covers under limb map m (its
// skipped range and, on the source side, its gap included)
long long span_limbs(int num_limbs, const chd_limb_map &m, bool src_side) {
  const long long top_logical =
      num_limbs - 1 + (m.skip_lo < num_limbs ? m.skip_len : 0);
  const long long gap = src_side ? std::max(m.src_gap, 0) : 0;
  return top_logical + 1 + gap;
}
// chd::sets_disjoint_words over polynomials of limbs_a / limbs_b limbs
bool sets_disjoint(const uint32_t *a, long long pstride_a, int num_a,
                   long long limbs_a, const uint32_t *b, long long pstride_b,
                   int num_b, long long limbs_b) {
  return sets_disjoint_words(a, pstride_a, num_a, limbs_a * kN, b, pstride_b,
                             num_b, limbs_b * kN);
}
// the ModDown epilogue operand src2 of num_polys polynomials: limbs
// [src2_lo, src2_hi) of the output read src2 limbs 0 .. src2_hi - src2_lo;
// true when none of them overlaps the destination polynomial at dst
bool src2_disjoint(const uint32_t *src2, long long src2_pstride,
                   int src2_lo, int src2_hi, int num_polys,
                   const uint32_t *dst, long long dst_limbs) {
  if (src2 == nullptr || src2_hi <= src2_lo) return true;
  return sets_disjoint(src2, src2_pstride, num_polys, src2_hi - src2_lo, dst,
                       0, 1, dst_limbs);
}
}  // namespace

namespace {
int ntt_fwd_common(const char *name, const chd_tables *t,
                   const chd_limb_map *m, uint32_t *dst,
                   long long dst_pstride, const uint32_t *src,
                   long long src_pstride, int num_limbs, int num_polys,
                   const uint32_t *pre_cst, void *stream, bool two_pass) {
  if (!t || !m || !dst || !src || num_limbs < 0 || num_polys < 0)
    return set_error(CHD_ERR_ARG, std::string(name) + ": invalid argument");
  NttArgs a{};
  a.fwd_two_pass = two_pass ? 1 : 0;
  a.src = src;
  a.dst = dst;
  a.src_pstride = src_pstride;
  a.dst_pstride = dst_pstride;
  a.map = *m;
  a.tab = *t;
  a.cst = pre_cst;
  a.src_disjoint =
      sets_disjoint(src, src_pstride, num_polys, span_limbs(num_limbs, *m, true),
                    dst, dst_pstride, num_polys,
                    span_limbs(num_limbs, *m, false))
          ? 1
          : 0;
  // the two passes run in place only when every limb is read from where it
  // is written: the same base, polynomial stride and limb layout
  if (!a.src_disjoint &&
      (src != dst || m->src_gap != 0 ||
       (num_polys > 1 && src_pstride != dst_pstride)))
    return set_error(CHD_ERR_ARG,
                     std::string(name) +
                         ": source and destination overlap without being the "
                         "same polynomials");
  hipError_t e = launch_ntt_fwd(a, num_limbs, num_polys, pre_cst != nullptr,
                                kEpiStore, static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return set_error(CHD_ERR_HIP,
                     std::string(name) + ": " + hipGetErrorString(e));
  return 0;
}
}  // namespace

extern "C" int chd_k_ntt_fwd(const chd_tables *t, const chd_limb_map *m,
                             uint32_t *dst, long long dst_pstride,
                             const uint32_t *src, long long src_pstride,
                             int num_limbs, int num_polys,
                             const uint32_t *pre_cst, void *stream) {
  return ntt_fwd_common("chd_k_ntt_fwd", t, m, dst, dst_pstride, src,
                        src_pstride, num_limbs, num_polys, pre_cst, stream,
                        false);
}

extern "C" int chd_k_ntt_fwd_2p(const chd_tables *t, const chd_limb_map *m,
                                uint32_t *dst, long long dst_pstride,
                                const uint32_t *src, long long src_pstride,
                                int num_limbs, int num_polys,
                                const uint32_t *pre_cst, void *stream) {
  return ntt_fwd_common("chd_k_ntt_fwd_2p", t, m, dst, dst_pstride, src,
                        src_pstride, num_limbs, num_polys, pre_cst, stream,
                        true);
}

#ifdef CHD_PHASE_TIMESTAMPS
// the instrumented build only: where ntt_fwd_1p's waves write their phase
// timestamps (8 words per wave, waves = 16 per workgroup); NULL stops them
extern "C" int chd_debug_phase_timestamps(unsigned long long *buf,
                                          int waves) {
  if (buf == nullptr) waves = 0;
  if (waves < 0) return set_error(CHD_ERR_ARG, "invalid wave count");
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_phase_ts), &buf, sizeof(buf)) !=
          hipSuccess ||
      hipMemcpyToSymbol(HIP_SYMBOL(g_phase_waves), &waves, sizeof(waves)) !=
          hipSuccess)
    return set_error(CHD_ERR_HIP, "chd_debug_phase_timestamps");
  return 0;
}
#endif

extern "C" int chd_k_ntt_fwd_moddown(const chd_tables *t,
                                     const chd_limb_map *m, uint32_t *dst,
                                     int num_limbs, const uint32_t *src2,
                                     int src2_lo, int src2_hi,
                                     const uint32_t *inv_prod,
                                     const uint32_t *pad, void *stream) {
  if (!t || !m || !dst || !inv_prod || num_limbs < 0 ||
      (src2 == nullptr && src2_hi > src2_lo) || src2 == dst)
    return set_error(CHD_ERR_ARG, "chd_k_ntt_fwd_moddown: invalid argument");
  if (!src2_disjoint(src2, 0, src2_lo, src2_hi, 1, dst,
                     span_limbs(num_limbs, *m, false)))
    return set_error(CHD_ERR_ARG,
                     "chd_k_ntt_fwd_moddown: src2 overlaps the destination");
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

static int ntt_inv_common(const char *name, const chd_tables *t,
                          const chd_limb_map *m, uint32_t *dst,
                          long long dst_pstride, const uint32_t *src,
                          const uint32_t *src_mul, long long src_pstride,
                          int num_limbs, int num_polys, const uint32_t *cst,
                          int centre, void *stream, bool one_pass = false) {
  if (!t || !m || !dst || !src || !cst || num_limbs < 0 || num_polys < 0 ||
      (one_pass && (src_mul != nullptr || t->twist == nullptr)))
    return set_error(CHD_ERR_ARG, std::string(name) + ": invalid argument");
  NttArgs a{};
  a.src = src;
  a.src_mul = src_mul;
  a.dst = dst;
  a.src_pstride = src_pstride;
  a.dst_pstride = dst_pstride;
  a.map = *m;
  a.tab = *t;
  a.cst = cst;
  a.src_disjoint =
      sets_disjoint(src, src_pstride, num_polys, span_limbs(num_limbs, *m, true),
                    dst, dst_pstride, num_polys,
                    span_limbs(num_limbs, *m, false))
          ? 1
          : 0;
  if (one_pass && !a.src_disjoint)
    return set_error(CHD_ERR_ARG,
                     std::string(name) +
                         ": the single pass needs a source apart from the "
                         "destination");
  a.inv_one_pass = one_pass ? 1 : 0;
  hipError_t e =
      launch_ntt_inv(a, num_limbs, num_polys,
                     centre ? kEpiConstCentre : kEpiConst,
                     static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return set_error(CHD_ERR_HIP,
                     std::string(name) + ": " + hipGetErrorString(e));
  return 0;
}

extern "C" int chd_k_ntt_inv(const chd_tables *t, const chd_limb_map *m,
                             uint32_t *dst, long long dst_pstride,
                             const uint32_t *src, long long src_pstride,
                             int num_limbs, int num_polys, const uint32_t *cst,
                             int centre, void *stream) {
  return ntt_inv_common("chd_k_ntt_inv", t, m, dst, dst_pstride, src, nullptr,
                        src_pstride, num_limbs, num_polys, cst, centre,
                        stream);
}

extern "C" int chd_k_ntt_inv_1p(const chd_tables *t, const chd_limb_map *m,
                                uint32_t *dst, long long dst_pstride,
                                const uint32_t *src, long long src_pstride,
                                int num_limbs, int num_polys,
                                const uint32_t *cst, int centre,
                                void *stream) {
  return ntt_inv_common("chd_k_ntt_inv_1p", t, m, dst, dst_pstride, src,
                        nullptr, src_pstride, num_limbs, num_polys, cst,
                        centre, stream, true);
}

extern "C" int chd_k_ntt_inv_cols(const chd_tables *t, const chd_limb_map *m,
                                  uint32_t *dst, long long dst_pstride,
                                  int num_limbs, int num_polys,
                                  const uint32_t *cst, int centre,
                                  void *stream) {
  if (!t || !m || !dst || !cst || num_limbs < 0 || num_polys < 0)
    return set_error(CHD_ERR_ARG, "chd_k_ntt_inv_cols: invalid argument");
  if (num_limbs == 0 || num_polys == 0) return 0;
  NttArgs a{};
  a.src = dst;
  a.dst = dst;
  a.src_pstride = dst_pstride;
  a.dst_pstride = dst_pstride;
  a.map = *m;
  a.map.src_gap = 0;
  a.tab = *t;
  a.cst = cst;
  hipError_t e = launch_ntt_inv_cols(a, num_limbs, num_polys,
                                     centre ? kEpiConstCentre : kEpiConst,
                                     static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return set_error(CHD_ERR_HIP, std::string("chd_k_ntt_inv_cols: ") +
                                      hipGetErrorString(e));
  return 0;
}

extern "C" int chd_k_ntt_inv_mul(const chd_tables *t, const chd_limb_map *m,
                                 uint32_t *dst, long long dst_pstride,
                                 const uint32_t *src, const uint32_t *src_mul,
                                 long long src_pstride, int num_limbs,
                                 int num_polys, const uint32_t *cst,
                                 int centre, void *stream) {
  if (src_mul == nullptr)
    return set_error(CHD_ERR_ARG, "chd_k_ntt_inv_mul: invalid argument");
  return ntt_inv_common("chd_k_ntt_inv_mul", t, m, dst, dst_pstride, src,
                        src_mul, src_pstride, num_limbs, num_polys, cst,
                        centre, stream);
}

extern "C" int chd_k_ntt_fwd_groups(const chd_tables *t, const chd_limb_map *m,
                                    uint32_t *modup, long long group_stride,
                                    int num_groups, int alpha, int group_shift,
                                    int group_limbs, int with_rows,
                                    void *stream) {
  return chd_k_ntt_fwd_groups_batch(t, m, modup, group_stride, num_groups, 1,
                                    alpha, group_shift, group_limbs,
                                    with_rows, stream);
}

extern "C" int chd_k_ntt_fwd_groups_batch(
    const chd_tables *t, const chd_limb_map *m, uint32_t *modup,
    long long group_stride, int num_groups, int num_inputs, int alpha,
    int group_shift, int group_limbs, int with_rows, void *stream) {
  if (!t || !m || !modup || group_limbs < m->num_q || num_inputs < 1 ||
      num_inputs > CHD_MAX_JOBS ||
      !groups_valid(num_groups, alpha, group_shift, m->num_q))
    return set_error(CHD_ERR_ARG, "chd_k_ntt_fwd_groups: invalid argument");
  NttArgs a{};
  a.group_period = num_groups;
  a.src = modup;
  a.dst = modup;
  a.src_pstride = group_stride;
  a.dst_pstride = group_stride;
  a.map = *m;
  a.map.src_gap = 0;
  a.tab = *t;
  a.group_alpha = alpha;
  a.group_shift = group_shift;
  a.group_limbs = group_limbs;
  // grid.y covers the largest group (the smallest skip range)
  int min_skip = alpha;
  for (int g = 0; g < num_groups; g++)
    min_skip = std::min(min_skip, group_hi(g, alpha, group_shift, m->num_q) -
                                      group_lo(g, alpha, group_shift));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nz = num_groups * num_inputs;
  hipError_t e = launch_ntt_fwd_cols(a, group_limbs - min_skip, nz, s);
  if (e == hipSuccess && with_rows)
    e = launch_ntt_fwd_rows(a, group_limbs - min_skip, nz, s);
  if (e != hipSuccess)
    return set_error(CHD_ERR_HIP, std::string("chd_k_ntt_fwd_groups: ") +
                                      hipGetErrorString(e));
  return 0;
}

namespace {
const char *keyacc_job_error(const chd_keyacc_args *a) {
  const bool tensor = a->a1 != nullptr;
  if (!a->modup || !a->p_prod || !a->acc_b || !a->acc_a || a->alpha < 1 ||
      (tensor ? !a->b1 || !a->b2 || !a->a2 : !a->d) ||
      a->beta > CHD_MAX_JOBS ||
      !groups_valid(a->beta, a->alpha, a->group_shift, a->num_q))
    return "invalid argument";
  for (int g = 0; g < a->beta; g++)
    if (!a->kb[g] || !a->ka[g]) return "null key pointer";
  if ((a->intt_b == nullptr) != (a->intt_a == nullptr) ||
      (a->intt_b != nullptr &&
       (a->intt_lo < 0 || a->intt_lo >= a->num_q + a->alpha)))
    return "invalid INTT output";
  return nullptr;
}
}  // namespace

extern "C" int chd_k_modup_keyacc(const chd_tables *t,
                                  const chd_keyacc_args *args, void *stream) {
  return chd_k_modup_keyacc_batch(t, args, 1, stream);
}

extern "C" int chd_k_modup_keyacc_batch(const chd_tables *t,
                                        const chd_keyacc_args *jobs,
                                        int num_jobs, void *stream) {
  if (!t || !jobs || num_jobs < 1 || num_jobs > CHD_MAX_JOBS)
    return set_error(CHD_ERR_ARG, "chd_k_modup_keyacc: invalid argument");
  KeyAccBatch b{};
  b.tab = *t;
  for (int j = 0; j < num_jobs; j++) {
    if (const char *err = keyacc_job_error(&jobs[j]))
      return set_error(CHD_ERR_ARG, std::string("chd_k_modup_keyacc: ") + err);
    // one grid covers every job: the limb ranges must agree
    if (jobs[j].num_q != jobs[0].num_q || jobs[j].alpha != jobs[0].alpha)
      return set_error(CHD_ERR_ARG,
                       "chd_k_modup_keyacc: jobs of different levels");
    b.job[j] = jobs[j];
  }
  hipError_t e =
      launch_modup_keyacc(b, num_jobs, static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return set_error(CHD_ERR_HIP, std::string("chd_k_modup_keyacc: ") +
                                      hipGetErrorString(e));
  return 0;
}

namespace {
// NttArgs of a batched ModDown NTT: destinations, the epilogue operand src2
// and its constants, after the checks both entry points share
int moddown_multi_args(const char *who, const chd_tables *t,
                       const chd_limb_map *m, uint32_t *const *dst,
                       int num_polys, int num_limbs, const uint32_t *src2,
                       long long src2_pstride, int src2_lo, int src2_hi,
                       const uint32_t *inv_prod, const uint32_t *pad,
                       NttArgs *out) {
  if (!t || !m || !dst || !inv_prod || num_limbs < 0 || num_polys < 1 ||
      num_polys > CHD_MAX_JOBS || (src2 == nullptr && src2_hi > src2_lo))
    return set_error(CHD_ERR_ARG, std::string(who) + ": invalid argument");
  NttArgs &a = *out;
  a = NttArgs{};
  for (int p = 0; p < num_polys; p++) {
    if (!dst[p])
      return set_error(CHD_ERR_ARG,
                       std::string(who) + ": invalid destination");
    // every workgroup reads src2 while others write: no overlap at all
    if (!src2_disjoint(src2, src2_pstride, src2_lo, src2_hi, num_polys,
                       dst[p], span_limbs(num_limbs, *m, false)))
      return set_error(CHD_ERR_ARG,
                       std::string(who) + ": src2 overlaps a destination");
    a.dst_list[p] = dst[p];
  }
  a.src = dst[0];
  a.dst = dst[0];
  a.map = *m;
  a.map.src_gap = 0;
  a.tab = *t;
  a.src2 = src2;
  a.src2_pstride = src2_pstride;
  a.src2_lo = src2_lo;
  a.src2_hi = src2_hi;
  a.cst2 = inv_prod;
  a.pad = pad;
  return 0;
}
}  // namespace

extern "C" int chd_k_ntt_fwd_moddown_multi(
    const chd_tables *t, const chd_limb_map *m, uint32_t *const *dst,
    int num_polys, int num_limbs, const uint32_t *src, long long src_pstride,
    const uint32_t *src2, long long src2_pstride, int src2_lo, int src2_hi,
    const uint32_t *inv_prod, const uint32_t *pad, void *stream) {
  NttArgs a;
  if (int st = moddown_multi_args("chd_k_ntt_fwd_moddown_multi", t, m, dst,
                                  num_polys, num_limbs, src2, src2_pstride,
                                  src2_lo, src2_hi, inv_prod, pad, &a))
    return st;
  if (src != nullptr) {
    // separate source: single-pass kernel when no destination overlaps it
    bool ok = true;
    for (int p = 0; p < num_polys; p++)
      ok = ok && sets_disjoint(src, src_pstride, num_polys,
                               span_limbs(num_limbs, a.map, true), dst[p], 0,
                               1, span_limbs(num_limbs, a.map, false));
    if (!ok)
      return set_error(CHD_ERR_ARG,
                       "chd_k_ntt_fwd_moddown_multi: source overlaps a "
                       "destination");
    a.src = src;
    a.src_pstride = src_pstride;
    a.src_disjoint = 1;
  }
  hipError_t e = launch_ntt_fwd(a, num_limbs, num_polys, false, kEpiModDown,
                                static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return set_error(CHD_ERR_HIP, std::string("chd_k_ntt_fwd_moddown_multi: ") +
                                      hipGetErrorString(e));
  return 0;
}

extern "C" int chd_k_ntt_fwd_moddown_bconv1_multi(
    const chd_tables *t, const chd_limb_map *m, uint32_t *const *dst,
    int num_polys, int num_limbs, const int32_t *src1, long long src1_pstride,
    const uint32_t *bconv1, const uint32_t *src2, long long src2_pstride,
    int src2_lo, int src2_hi, const uint32_t *inv_prod, const uint32_t *pad,
    void *stream) {
  const char *who = "chd_k_ntt_fwd_moddown_bconv1_multi";
  if (!src1 || !bconv1)
    return set_error(CHD_ERR_ARG, std::string(who) + ": invalid argument");
  NttArgs a;
  if (int st = moddown_multi_args(who, t, m, dst, num_polys, num_limbs, src2,
                                  src2_pstride, src2_lo, src2_hi, inv_prod,
                                  pad, &a))
    return st;
  // each workgroup reads all of its polynomial's source limb while others
  // write their destinations: no overlap at all
  const uint32_t *s1 = reinterpret_cast<const uint32_t *>(src1);
  for (int p = 0; p < num_polys; p++)
    if (!sets_disjoint(s1, src1_pstride, num_polys, 1, dst[p], 0, 1,
                       span_limbs(num_limbs, a.map, false)))
      return set_error(CHD_ERR_ARG,
                       std::string(who) + ": source overlaps a destination");
  a.src = s1;
  a.src_pstride = src1_pstride;
  a.src_disjoint = 1;
  a.src_bcast = 1;
  a.cst = bconv1;
  hipError_t e = launch_ntt_fwd(a, num_limbs, num_polys, false, kEpiModDown,
                                static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return set_error(CHD_ERR_HIP,
                     std::string(who) + ": " + hipGetErrorString(e));
  return 0;
}
