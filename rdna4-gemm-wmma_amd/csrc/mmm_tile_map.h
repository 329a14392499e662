// Tile scheduling for the MI355X GEMM kernels: linear workgroup id -> output tile.
//
// Replaces the reference's block remap (mmm.cpp:1219-1236, mmmTensor.cpp:50-65), which
// groups tiles into column strips of 32 but is not a bijection when gridDim.x > 32 and
// gridDim.x % 32 != 0 (tiles are then skipped and others computed twice).
//
// This mapping is a bijection for every grid.  It is built from two bijective steps:
//  1. XCD compaction.  The command processor hands workgroups to the 8 XCDs round-robin
//     (workgroup b runs on XCD b % 8).  Each XCD has its own L2, so workgroups that share
//     operand panels should sit on the same XCD: virtual id v gives XCD x a contiguous
//     range of v.  With q = n / 8 and r = n % 8, XCDs 0..r-1 own q+1 ids and the rest q.
//  2. Grouped ordering.  Virtual ids walk GROUP_M tile-rows down a column before moving to
//     the next column, so 32 consecutive ids (one XCD's 32 CUs) form a 4 x 8 tile patch
//     that shares 4 A panels and 8 B panels in that XCD's L2.
#pragma once

#ifdef __HIPCC__
#define MMM_HD __host__ __device__ __forceinline__
#else
#define MMM_HD inline
#endif

namespace mmm {

constexpr int kNumXcd = 8;

MMM_HD int xcd_compact(int b, int n) {
  const int q = n / kNumXcd, r = n % kNumXcd;
  const int x = b % kNumXcd, slot = b / kNumXcd;
  return (x < r) ? x * (q + 1) + slot : r * (q + 1) + (x - r) * q + slot;
}

MMM_HD void grouped_tile(int v, int tiles_m, int tiles_n, int group_m, int* tm, int* tn) {
  const int per_group = group_m * tiles_n;
  const int g = v / per_group;
  const int first_m = g * group_m;
  const int rows = (tiles_m - first_m < group_m) ? (tiles_m - first_m) : group_m;
  const int w = v % per_group;
  *tm = first_m + w % rows;
  *tn = w / rows;
}

MMM_HD void tile_of_block(int b, int tiles_m, int tiles_n, int group_m, int* tm, int* tn) {
  grouped_tile(xcd_compact(b, tiles_m * tiles_n), tiles_m, tiles_n, group_m, tm, tn);
}

}  // namespace mmm
