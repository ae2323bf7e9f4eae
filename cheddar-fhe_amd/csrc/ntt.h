// Internal (non-ABI) interface of the NTT kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cheddar_kernels.h"

namespace chd {

using NttTables = chd_tables;
using LimbMap = chd_limb_map;

enum NttEpilogue : int {
  kEpiStore = 0,     // canonical [0, q)
  kEpiModDown = 1,   // MontMul(MontMul(src2,pad) - y, cst2)
  kEpiConst = 2,     // MontMul(y, cst)
  kEpiConstCentre = 3,
};

struct NttArgs {
  const uint32_t *src;
  uint32_t *dst;
  long long src_pstride;  // words between polynomials (grid.z)
  long long dst_pstride;
  LimbMap map;
  NttTables tab;
  const uint32_t *cst;    // per-limb MontMul constant (prologue or epilogue)
  // inverse row pass only: when set, the input element is the canonical
  // MontMul(src, src_mul) (same layout as src)
  const uint32_t *src_mul;
  // ModDown epilogue (src/core/NTT.cu:456-601)
  const uint32_t *src2;   // kept limbs of the original input
  long long src2_pstride;
  int src2_lo, src2_hi;   // logical limb range that src2 covers
  const uint32_t *cst2;   // inv prime product per logical limb
  const uint32_t *pad;    // optional padding per src2 limb (nullptr: none)
  // ModUp group mode (group_alpha > 0): grid.z = dnum group g, whose own
  // limbs [group_lo(g), group_hi(g)) are skipped; every group holds
  // group_limbs logical limbs (NTTForModUp for all groups in one launch)
  int group_alpha;
  int group_shift;
  int group_limbs;
  // with several inputs in group mode, grid.z runs over (input, group) and
  // the group is blockIdx.z % group_period (0: blockIdx.z)
  int group_period;
  // optional per-polynomial base pointers (used instead of base + z*stride
  // when dst_list[0] is set): polynomials in separate allocations
  uint32_t *dst_list[CHD_MAX_JOBS];
  // forward only: the source limbs do not overlap the destination, so the
  // single-pass kernel (which reads every quarter of a limb while writing
  // its own) may run
  int src_disjoint;
  // inverse only: run the single pass over residue classes (src_disjoint
  // set, no src_mul, tab.twist present; checked by the caller)
  int inv_one_pass;
  // forward only: run the two passes even where the single pass would
  int fwd_two_pass;
  // single-pass ModDown NTT only: every limb of polynomial z reads the one
  // centred source limb src + z * src_pstride, times its cst[l] (a
  // one-source BConv fused into the transform's first round)
  int src_bcast;
};

// Fused ModUp row pass + evaluation-key inner product (PAccum) + CAccum for
// up to CHD_MAX_JOBS independent key switches of one level (grid.z = job).
struct KeyAccBatch {
  chd_tables tab;
  chd_keyacc_args job[CHD_MAX_JOBS];
};
hipError_t launch_modup_keyacc(const KeyAccBatch &a, int num_jobs,
                               hipStream_t s);

// Forward NTT over grid (limbs, polys); pre_const multiplies the input by
// MontMul(x, cst[limb]) first (Montgomery conversion).
hipError_t launch_ntt_fwd(const NttArgs &a, int num_limbs, int num_polys,
                          bool pre_const, int epilogue, hipStream_t s);
// Inverse NTT (kernels compute N * intt; the N^-1 is in the constant)
// the inverse's second pass alone (in place on a.dst)
hipError_t launch_ntt_inv_cols(const NttArgs &a, int num_limbs, int num_polys,
                               int epilogue, hipStream_t s);
hipError_t launch_ntt_inv(const NttArgs &a, int num_limbs, int num_polys,
                          int epilogue, hipStream_t s);
// column pass only (ModUp group mode uses grid.z = groups)
hipError_t launch_ntt_fwd_cols(const NttArgs &a, int num_limbs, int num_z,
                               hipStream_t s);
hipError_t launch_ntt_fwd_rows(const NttArgs &a, int num_limbs, int num_z,
                               hipStream_t s);

}  // namespace chd
