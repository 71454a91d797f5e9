// Helpers shared by the GEMM kernels.
#pragma once

#include "common.h"

namespace cgpt {

#ifndef CGPT_GROUP_M
#define CGPT_GROUP_M 8
#endif
constexpr int kGroupM = CGPT_GROUP_M;
constexpr int kNumXcd = 8;
constexpr uint32_t kBufferRsrcWord3 = 0x00020000u;  // raw buffer, gfx9 family

// Map a hardware block (or persistent tile) id to (tile_m, tile_n):
// XCD-contiguous ranges of logical tiles, then groups of kGroupM tile rows.
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int nblocks = tiles_m * tiles_n;
  const int q = nblocks / kNumXcd, r = nblocks % kNumXcd;
  const int xcd = bid % kNumXcd;
  const int logical = xcd * q + (xcd < r ? xcd : r) + bid / kNumXcd;
  const int group = kGroupM * tiles_n;
  const int g = logical / group;
  const int first_m = g * kGroupM;
  const int gsz = min(tiles_m - first_m, kGroupM);
  const int in_group = logical % group;
  tm = first_m + in_group % gsz;
  tn = in_group / gsz;
}

}  // namespace cgpt
