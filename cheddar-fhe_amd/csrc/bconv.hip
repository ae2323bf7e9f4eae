// BConv: the base-conversion matrix product of ModUp / ModDown / Rescale
// (reference kernel ModSwitchMatrixMult, src/core/ModSwitch.cu:23-171),
// on the int8 matrix cores.
//
//   dst[pos(k)][n] = sum_i c_i[n] * T[k][i] * 2^-32  mod p_k
//
// c_i are centred int32 residues (the INTT epilogue's output, |c| < 2^30) and
// T is the reference's "double Montgomery" table centre(qhat_i R^2 mod p_k).
//
// Byte-digit decomposition. The host expands the table over the four byte
// positions of a source: V[k][(i,b)] = centre(T[k][i] 256^b mod p_k). A
// centred source c splits into signed digits d_0..d_3 in [-128, 127] with
// c = sum_b d_b 256^b; the packed word (c + 0x808080) ^ 0x808080 holds exactly
// those four int8 digits, so a source costs two VALU ops to decompose. V is
// split the same way into digit planes v_0..v_3 (packed on the host). Then
//
//   acc_c[n][k] = sum_{(i,b)} d_b(c_i[n]) v_c[k][(i,b)]      (int8 MFMA, K=64)
//   dst[k][n]   = (acc_0 + 2^8 acc_1 + 2^16 acc_2 + 2^24 acc_3) 2^-32 mod p_k
//
// which is congruent to sum_i c_i T[k][i] 2^-32. |acc_c| <= 64 * 128 * 128 =
// 2^20, so the planes pair up exactly in int32 (acc_0 + 2^8 acc_1 and
// acc_2 + 2^8 acc_3, each below 2^30), one 64-bit multiply-add joins the
// pairs exactly (< 2^47), and one signed Montgomery reduction (the
// reference's, Basic.cuh:72-88) gives the residue times 2^-32: the canonical
// result is bit-identical to the reference's for every input. The MFMA
// results are kept in VGPRs (the build passes -amdgpu-mfma-vgpr-form for
// this file).
//
// One v_mfma_i32_16x16x64_i8 multiplies a 16-coefficient x 64 (sources x
// bytes, zero-padded beyond 4 * src_len) tile by a 64 x 16-destination tile
// of one digit plane; more than 16 sources take a second K chunk of 64
// accumulated into the same tile (|acc| <= 2^21, still exact). Operand lanes (checked on gfx950): A row = lane % 16,
// k = 16 (lane / 16) + byte; B column = lane % 16, same k; D column =
// lane % 16, rows 4 (lane / 16) + 0..3. So lane l packs sources
// 4 (l / 16) .. + 3 of coefficient l % 16, and finishes four consecutive
// coefficients of destination 16 t + l % 16.
//
// Grid (N / kCoefPerBlock, destination tiles or 1, jobs), 256 threads; a wave
// takes kTilesPerWave 16-coefficient tiles. The packed table (4 KiB per 16 destinations and K
// chunk) is read through the caches by every wave.
#include <algorithm>
#include <cstring>
#include <vector>

#include "chd_device.h"
#include "cheddar_kernels.h"
#include "kernel_common.h"

namespace chd {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kChunkSrc = 16;          // 4 bytes x 16 sources = K of 64
constexpr int kMaxChunks = 2;
constexpr int kMaxSrc = kChunkSrc * kMaxChunks;
constexpr int kTilesPerWave = 2;
constexpr int kCoefPerBlock = (kThreads / 64) * kTilesPerWave * 16;
constexpr int kPlaneBytes = 64 * 16;   // one digit plane of a 16-dst tile
static_assert(kTilesPerWave == 2,
              "a packed last tile carries exactly the wave's two coefficient "
              "tiles, and a wave's 32 coefficients are one 128-byte line");
constexpr int kLdsRow = 36;  // words per LDS row: 32 coefficients + pad
constexpr int kFewJobs = 4;   // a batch of at most this many jobs: kFew
static_assert(kN == 256 * 256 && kCoefPerBlock == 4 * kTilesPerWave * 16 &&
                  kTilesPerWave * 16 == 32,
              "kFew maps the N / kCoefPerBlock workgroups onto 8 column tiles "
              "of 32 coefficients x 64 groups of four 256-coefficient rows");

// orders a wave's LDS writes before its reads of other lanes' words (a
// wave's LDS instructions execute in order; only the compiler must not move
// them)
__device__ __forceinline__ void wave_lds_sync_bc() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct BconvBatch {
  chd_bconv_job job[CHD_MAX_BCONV_JOBS];
};

// A job with at most 8 sources uses only K 0..31 of the MFMA (8 sources x 4
// bytes). When its last destination tile is at most half full (1..8 of 16
// destinations), that tile is "packed": the second K half carries a second
// group of 16 coefficients, and destination columns 8..15 repeat columns
// 0..7 for that group, so no lane of the tile computes a dead destination:
//   A row r = [coefficient n_wave + r, K 0..31 | coefficient n_wave + 16 + r,
//              K 32..63]
//   B column c < 8 = [V(16 t + c) | 0],  column c >= 8 = [0 | V(16 t + c - 8)]
// The host table layout and the kernel both follow this rule.
__host__ __device__ __forceinline__ bool packed_last_tile(int src_len,
                                                         int dst_len) {
  const int rem = dst_len & 15;
  return src_len <= 8 && rem != 0 && rem <= 8;
}

// four signed byte digits of a centred value |c| < 2^30, packed as int8 x4
__device__ __forceinline__ int digits(int32_t c) {
  return static_cast<int>((static_cast<uint32_t>(c) + 0x808080u) ^ 0x808080u);
}

// the four digit planes of destination tile tt, K chunk ch (zero beyond the
// job's chunks)
template <int kChunks>
__device__ __forceinline__ void load_planes(v4i (&bp)[kChunks][4],
                                            const v4i *__restrict__ tab,
                                            int tt, int nk, int lane) {
#pragma unroll
  for (int ch = 0; ch < kChunks; ch++) {
    if (ch < nk) {
      const v4i *tp = tab + (static_cast<size_t>(tt * nk + ch) * 4) * 64 + lane;
      bp[ch][0] = tp[0];
      bp[ch][1] = tp[64];
      bp[ch][2] = tp[128];
      bp[ch][3] = tp[192];
    } else {
      const v4i z = {0, 0, 0, 0};
      bp[ch][0] = bp[ch][1] = bp[ch][2] = bp[ch][3] = z;
    }
  }
}

template <int kChunks, bool kStream, bool kFew>
__global__ __launch_bounds__(kThreads) void bconv_mfma(chd_tables t,
                                                       chd_limb_map m,
                                                       BconvBatch b) {
  __shared__ __align__(16) uint32_t lds[(kThreads / 64) * 16 * kLdsRow];
  // the job by value: its fields stay in scalar registers
  const chd_bconv_job jb = b.job[blockIdx.z];
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int wave = threadIdx.x >> 6;
  // a wave's 32 coefficients: 128 consecutive ones per workgroup, or with
  // kFew (a batch of a few jobs, one generation of workgroups) four rows of
  // one 32-coefficient column tile, so that the workgroup runs on the XCD
  // (block id mod 8) of the column-pass workgroups that write its sources
  // and read its output
  const int n_wave =
      kFew ? (((static_cast<int>(blockIdx.x) >> 3) * 4 + wave) << 8) +
                 (static_cast<int>(blockIdx.x) & 7) * (kTilesPerWave * 16)
           : blockIdx.x * kCoefPerBlock + wave * kTilesPerWave * 16;
  const int32_t *__restrict__ src = jb.src;
  const v4i *__restrict__ tab = static_cast<const v4i *>(jb.table);
  // this job's K chunks (its table holds exactly that many per tile)
  const int nk = kChunks == 1 ? 1 : (jb.src_len + kChunkSrc - 1) / kChunkSrc;
  const int tiles = (jb.dst_len + 15) >> 4;
  // the grid covers the batch's largest job; a smaller one has fewer tiles
  if (static_cast<int>(blockIdx.y) >= tiles) return;
  // at most 8 sources: lanes 32..63 (K 32..63, zero rows of B in the other
  // tiles) hold the sources of the second coefficient group instead
  const bool narrow = jb.src_len <= 8;
  const bool packed = packed_last_tile(jb.src_len, jb.dst_len);
  // Source words of this wave's coefficient tiles, per K chunk. Every load
  // is issued (sources beyond src_len read the last source and are zeroed
  // after), so they are all in flight together instead of one guarded load
  // at a time.
  int32_t cw[kChunks][kTilesPerWave][4];
  int si[kChunks][4];  // source index of each word (the same for both mt)
#pragma unroll
  for (int ch = 0; ch < kChunks; ch++)
#pragma unroll
    for (int mt = 0; mt < kTilesPerWave; mt++) {
      const bool second = ch == 0 && narrow && g >= 2;
      const int n = n_wave + (mt == 1 || second ? 16 : 0) + r;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int i = ch == 0 && narrow ? 4 * (g & 1) + j
                                        : kChunkSrc * ch + 4 * g + j;
        si[ch][j] = i;
        const int ic = min(i, jb.src_len - 1);
        cw[ch][mt][j] = src[(static_cast<size_t>(ic) << kLogN) + n];
      }
    }
  // prime of this lane's destination in tile tt (dead lanes beyond dst_len
  // take the last destination's: their results are not stored); the packed
  // tile's column c stands for destination 16 t + (c & 7)
  auto prime_of = [&](int tt, uint32_t &p, int32_t &pinv, int &pos) {
    const int col = packed && tt == tiles - 1 ? (r & 7) : r;
    const int kc = min(tt * 16 + col, jb.dst_len - 1);
    pos = kc + (kc >= jb.skip_lo ? jb.skip_len : 0);
    const bool aux = pos >= m.num_q;
    const int ti = m.tab_off + pos + (aux ? m.tab_gap : 0);
    p = t.q[ti];
    pinv = t.qinv[ti];
  };
  // A operands (the sources' signed digits), shared by every destination
  // tile this workgroup computes
  v4i a[kChunks][kTilesPerWave];
#pragma unroll
  for (int ch = 0; ch < kChunks; ch++)
#pragma unroll
    for (int mt = 0; mt < kTilesPerWave; mt++)
#pragma unroll
      for (int j = 0; j < 4; j++)
        a[ch][mt][j] = digits(si[ch][j] < jb.src_len ? cw[ch][mt][j] : 0);
  // the workgroup's destination tiles: blockIdx.y, then every gridDim.y-th
  // (a single conversion has a workgroup per tile, a batch one workgroup
  // for all of a job's tiles); each tile's primes and planes
  for (int tt = blockIdx.y; tt < tiles; tt += gridDim.y) {
  uint32_t p;
  int32_t pinv;
  int pos;
  prime_of(tt, p, pinv, pos);
  v4i bp[kChunks][4];
  load_planes<kChunks>(bp, tab, tt, nk, lane);
  // Recombination of the four planes of one MFMA output (4 coefficients of
  // one destination): pairs of planes in int32 (|acc_c| <= 2^21, so |lo|,
  // |hi| < 2^30), one 64-bit multiply-add y = lo + 2^16 hi (|y| < 2^47, far
  // inside the (-p 2^31, p 2^31) a signed Montgomery reduction takes),
  // reduced to y 2^-32 in (-p, p), then made canonical.
  auto finish = [&](const v4i (&d)[4]) {
    v4u o;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int32_t lo = d[0][i] + d[1][i] * 256;
      const int32_t hi = d[2][i] + d[3][i] * 256;
      const int64_t y = static_cast<int64_t>(hi) * 65536 + lo;
      const uint32_t u = static_cast<uint32_t>(mont_reduce_lazy(y, p, pinv));
      const uint32_t up = u + p;
      o[i] = u < up ? u : up;  // unsigned min: u + p when negative
    }
    return o;
  };
  // Results go out through this wave's LDS tile, [destination column][32
  // coefficients] (rows padded to 36 words), so that 8 lanes store the 128
  // contiguous bytes of one destination limb: each store instruction writes
  // 8 whole lines instead of 16 half lines. Inside a key switch (the batch
  // entry) the next launch, the NTT, reads the result right away, so it is
  // written with default (temporal) stores and stays in the caches (3 %
  // faster per HMult than streaming stores, measured); a standalone
  // conversion (kStream) writes with the streaming hint.
  uint32_t *xt = lds + wave * (16 * kLdsRow);
  auto store_rows = [&](int dst_base, int rows) {
    // rows destinations (8 or 16) of this tile, 8 per store instruction;
    // dst_base is the destination index of LDS row 0
    wave_lds_sync_bc();
#pragma unroll
    for (int h = 0; h < 2; h++) {
      if (h * 8 >= rows) break;
      const int row = h * 8 + (lane >> 3);
      const int piece = lane & 7;
      const v4u v = *reinterpret_cast<const v4u *>(xt + row * kLdsRow +
                                                  4 * piece);
      const int k = dst_base + row;
      if (k < jb.dst_len) {
        const int kp = k + (k >= jb.skip_lo ? jb.skip_len : 0);
        v4u *dp = reinterpret_cast<v4u *>(
            jb.dst + (static_cast<size_t>(kp) << kLogN) + n_wave + 4 * piece);
        if constexpr (kStream)
          __builtin_nontemporal_store(v, dp);
        else
          *dp = v;
      }
    }
  };
  if (!(packed && tt == tiles - 1)) {
    v4i d[kTilesPerWave][4];
#pragma unroll
    for (int mt = 0; mt < kTilesPerWave; mt++)
#pragma unroll
      for (int pl = 0; pl < 4; pl++) {
        const v4i z = {0, 0, 0, 0};
        d[mt][pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[0][mt], bp[0][pl],
                                                          z, 0, 0, 0);
#pragma unroll
        for (int ch = 1; ch < kChunks; ch++)
          d[mt][pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
              a[ch][mt], bp[ch][pl], d[mt][pl], 0, 0, 0);
      }
    // lane: destination column r, coefficients 16 mt + 4 g .. + 3
#pragma unroll
    for (int mt = 0; mt < kTilesPerWave; mt++)
      *reinterpret_cast<v4u *>(xt + r * kLdsRow + 16 * mt + 4 * g) =
          finish(d[mt]);
    store_rows(tt * 16, 16);
  } else {
    // the packed last tile, both coefficient groups at once (one K chunk:
    // nk is 1 for at most 8 sources): column r is destination
    // 16 tt + (r & 7) for coefficient group r >> 3
    v4i d[4];
#pragma unroll
    for (int pl = 0; pl < 4; pl++) {
      const v4i z = {0, 0, 0, 0};
      d[pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[0][0], bp[0][pl], z, 0,
                                                    0, 0);
    }
    *reinterpret_cast<v4u *>(xt + (r & 7) * kLdsRow + 16 * (r >> 3) +
                             4 * g) = finish(d);
    store_rows(tt * 16, 8);
  }
  // the next tile rewrites this wave's LDS tile after its lanes' reads
  wave_lds_sync_bc();
  }
}

// centred residue of v mod p
int64_t centre_mod(int64_t v, int64_t p) {
  v %= p;
  if (v < 0) v += p;
  if (v > p / 2) v -= p;
  return v;
}

}  // namespace
}  // namespace chd

using namespace chd;

extern "C" long long chd_bconv_table_size(int src_len, int dst_len) {
  if (src_len < 1 || src_len > kMaxSrc || dst_len < 1) return 0;
  const int nk = (src_len + kChunkSrc - 1) / kChunkSrc;
  return static_cast<long long>((dst_len + 15) / 16) * nk * 4 * kPlaneBytes;
}

extern "C" int chd_bconv_table_pack(void *host_out, const int32_t *table_ref,
                                    const uint32_t *dst_primes, int src_len,
                                    int dst_len) {
  if (!host_out || !table_ref || !dst_primes || src_len < 1 ||
      src_len > kMaxSrc || dst_len < 1)
    return set_error(CHD_ERR_ARG, "chd_bconv_table_pack: invalid argument");
  const int tiles = (dst_len + 15) / 16;
  const int nk = (src_len + kChunkSrc - 1) / kChunkSrc;
  const bool packed = packed_last_tile(src_len, dst_len);
  int8_t *out = static_cast<int8_t *>(host_out);
  std::memset(out, 0, static_cast<size_t>(tiles) * nk * 4 * kPlaneBytes);
  for (int k = 0; k < dst_len; k++) {
    const int64_t p = dst_primes[k];
    const int tt = k / 16, col = k % 16;
    // a packed last tile holds each destination twice: column col with K
    // 0..31 and column col + 8 with K 32..63
    const int copies = packed && tt == tiles - 1 ? 2 : 1;
    for (int i = 0; i < src_len; i++) {
      // the reference's table entry T itself: the kernel's Montgomery
      // reduction supplies the 2^-32
      const int64_t u = centre_mod(table_ref[static_cast<size_t>(k) * src_len + i], p);
      int64_t ub = u < 0 ? u + p : u;  // T * 256^b, canonical
      for (int bb = 0; bb < 4; bb++) {
        const int64_t v = centre_mod(ub, p);  // |v| < 2^30
        // signed digits of v: (v + 0x808080) has unsigned low bytes e_0..e_2
        // and a signed top byte e_3; digit b = e_b - 128 (b < 3), e_3
        const int64_t w = v + 0x808080;
        int8_t dig[4];
        for (int c = 0; c < 3; c++)
          dig[c] = static_cast<int8_t>(((w >> (8 * c)) & 0xff) - 128);
        dig[3] = static_cast<int8_t>(w >> 24);
        // K index of (i, bb): its chunk, and its lane / byte in that
        // chunk's B operand
        for (int cp = 0; cp < copies; cp++) {
          const int kk = 4 * i + bb + 32 * cp;
          const int ch = kk / 64;
          const int lane = ((kk % 64) / 16) * 16 + col + 8 * cp;
          const int byte = kk % 16;
          for (int c = 0; c < 4; c++)
            out[(((static_cast<size_t>(tt) * nk + ch) * 4 + c) * 64 + lane) *
                    16 +
                byte] = dig[c];
        }
        ub = (ub * 256) % p;
      }
    }
  }
  return 0;
}

namespace {
int launch_bconv(const chd_tables *t, const chd_limb_map *m,
                 const chd_bconv_job *jobs, int num_jobs, bool stream_out,
                 void *stream) {
  if (!t || !m || !jobs || num_jobs < 1 || num_jobs > CHD_MAX_BCONV_JOBS)
    return set_error(CHD_ERR_ARG, "chd_k_bconv_batch: invalid argument");
  BconvBatch b{};
  for (int j = 0; j < num_jobs; j++) {
    const chd_bconv_job &jb = jobs[j];
    if (!jb.dst || !jb.src || !jb.table || jb.src_len < 1 ||
        jb.src_len > kMaxSrc || jb.dst_len < 1 || jb.skip_len < 0)
      return set_error(CHD_ERR_ARG, "chd_k_bconv_batch: invalid job");
    b.job[j] = jb;
  }
  int max_src = 0, max_tiles = 0;
  for (int j = 0; j < num_jobs; j++) {
    max_src = std::max(max_src, jobs[j].src_len);
    max_tiles = std::max(max_tiles, (jobs[j].dst_len + 15) / 16);
  }
  // A single conversion: one destination tile per workgroup (blockIdx.y),
  // the coefficient blocks of a tile consecutive block ids, so the tiles of
  // one coefficient block land on the same XCD (kN / kCoefPerBlock is a
  // multiple of 8), whose L2 keeps the sources for them (config 3, 1,536
  // workgroups). A batch (key-switch ModUp and ModDown, at least 2 jobs)
  // already has enough workgroups: each one computes all of its job's tiles
  // from one load of the sources (the hoisted config-5 batches of 8 to 24
  // jobs 25.9 -> 23.4 us per launch on average, HMult's 8.7 -> 8.0 us;
  // walking two or four coefficient blocks per workgroup as well was
  // slower, 27.0 and 29.3 us).
  //
  // A batch of at most kFewJobs jobs (one key switch's ModUp or ModDown)
  // maps its workgroups onto the column tiles of the NTT passes around it
  // (kFew): about 1 us less per HMult with merged rescale at L = 4, 20 and
  // 24 (53.4-53.6 against 54.4-54.5, 87.6-88.3 against 88.6-89.8,
  // 90.2-90.3 against 91.0-91.3 us; three A/B pairs in one call); the
  // larger hoisting batches measured 0.6 % slower with that mapping and
  // keep the consecutive one.
  dim3 g(kN / kCoefPerBlock, num_jobs >= 2 ? 1 : max_tiles, num_jobs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool few = num_jobs >= 2 && num_jobs <= kFewJobs;
  if (max_src <= kChunkSrc) {
    if (stream_out)
      hipLaunchKernelGGL((bconv_mfma<1, true, false>), g, dim3(kThreads), 0, s, *t, *m, b);
    else if (few)
      hipLaunchKernelGGL((bconv_mfma<1, false, true>), g, dim3(kThreads), 0, s, *t, *m, b);
    else
      hipLaunchKernelGGL((bconv_mfma<1, false, false>), g, dim3(kThreads), 0, s, *t, *m, b);
  } else {
    if (stream_out)
      hipLaunchKernelGGL((bconv_mfma<2, true, false>), g, dim3(kThreads), 0, s, *t, *m, b);
    else if (few)
      hipLaunchKernelGGL((bconv_mfma<2, false, true>), g, dim3(kThreads), 0, s, *t, *m, b);
    else
      hipLaunchKernelGGL((bconv_mfma<2, false, false>), g, dim3(kThreads), 0, s, *t, *m, b);
  }
  return check_launch("chd_k_bconv_batch");
}
}  // namespace

extern "C" int chd_k_bconv_batch(const chd_tables *t, const chd_limb_map *m,
                                 const chd_bconv_job *jobs, int num_jobs,
                                 void *stream) {
  return launch_bconv(t, m, jobs, num_jobs, false, stream);
}

extern "C" int chd_k_bconv(const chd_tables *t, const chd_limb_map *m,
                           uint32_t *dst, const int32_t *src, int src_len,
                           int dst_len, const void *table, void *stream) {
  if (!t || !m || !dst || !src || !table || src_len < 1 ||
      src_len > kMaxSrc || dst_len < 1)
    return set_error(CHD_ERR_ARG, "chd_k_bconv: invalid argument");
  chd_bconv_job j{dst, src, table, src_len, dst_len, m->skip_lo, m->skip_len};
  return launch_bconv(t, m, &j, 1, true, stream);
}
