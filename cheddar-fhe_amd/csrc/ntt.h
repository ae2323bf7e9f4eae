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
  // ModDown epilogue (src/core/NTT.cu:456-601)
  const uint32_t *src2;   // kept limbs of the original input
  long long src2_pstride;
  int src2_lo, src2_hi;   // logical limb range that src2 covers
  const uint32_t *cst2;   // inv prime product per logical limb
  const uint32_t *pad;    // optional padding per src2 limb (nullptr: none)
};

// Forward NTT over grid (limbs, polys); pre_const multiplies the input by
// MontMul(x, cst[limb]) first (Montgomery conversion).
hipError_t launch_ntt_fwd(const NttArgs &a, int num_limbs, int num_polys,
                          bool pre_const, int epilogue, hipStream_t s);
// Inverse NTT (kernels compute N * intt; the N^-1 is in the constant)
hipError_t launch_ntt_inv(const NttArgs &a, int num_limbs, int num_polys,
                          int epilogue, hipStream_t s);

}  // namespace chd
