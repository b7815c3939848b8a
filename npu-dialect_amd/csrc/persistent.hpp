// persistent.hpp -- shared pieces of the persistent (tile-walking) kernels.
//
// A persistent kernel launches as many workgroups as the CUs can hold at
// once; each loads what every tile needs (filter fragments, requant
// parameters) once, then walks its share of the tiles, fetching the next
// tile's inputs into registers while the current tile is computed.
//
// Workgroups are dispatched round-robin over the 8 XCDs (blockIdx.x % 8), and
// each XCD has its own L2.  The tiles are split into 8 contiguous ranges, one
// per XCD, so tiles that share input rows (halos) run on the same L2.
#pragma once
#include <hip/hip_runtime.h>

#include "plans.hpp"

namespace npu {

constexpr int kXcds = 8;

struct TileWalk {
  int first, end, step;
};

// Tiles of this workgroup: first, first + step, ... below end.  gridDim.x must
// be a multiple of kXcds.
__device__ __forceinline__ TileWalk tile_walk(int ntiles) {
  const int xcd = blockIdx.x % kXcds;
  TileWalk w;
  w.step = gridDim.x / kXcds;
  w.end = (int)((long long)(xcd + 1) * ntiles / kXcds);
  w.first = (int)((long long)xcd * ntiles / kXcds) + blockIdx.x / kXcds;
  return w;
}

// Balanced contiguous share of `nrows` work rows for this workgroup: the
// workgroups of one XCD take neighbouring ranges (so rows that two ranges
// share are read through the same L2), and range sizes differ by at most
// one row, so no CU carries a whole extra tile.  gridDim.x must be a
// multiple of kXcds.
struct RowRange {
  int first, end;
};
__device__ __forceinline__ RowRange row_range(int nrows) {
  const int g = (blockIdx.x % kXcds) * (gridDim.x / kXcds) + blockIdx.x / kXcds;
  RowRange r;
  r.first = (int)((long long)nrows * g / gridDim.x);
  r.end = (int)((long long)nrows * (g + 1) / gridDim.x);
  return r;
}

// 2-D XCD blocks for a launch of one workgroup per output tile: the
// tiles_m x tiles_n tile grid cut into an xm x (8 / xm) grid of blocks,
// block x on XCD x (= blockIdx.x % 8), tiles taken N-major within a block,
// so an XCD reads only its block's rows of A and columns of B.  The grid is
// exactly tiles_m * tiles_n workgroups (xcd_block_grid picks xm so that the
// blocks divide the tile grid).
__device__ __forceinline__ void xcd_block_tile(int tiles_m, int tiles_n, int xm, int &tm, int &tn) {
  const int x = blockIdx.x % kXcds, l = blockIdx.x / kXcds;
  const int xn = kXcds / xm, rm = tiles_m / xm, rn = tiles_n / xn;
  tm = (x / xn) * rm + l % rm;
  tn = (x % xn) * rn + l / rm;
}

// The xm (1, 2, 4 or 8, dividing tiles_m, with 8 / xm dividing tiles_n) for
// xcd_block_tile whose blocks read the fewest A rows plus B columns per XCD
// (bm rows per tile row, bn_cols per tile column), or 0 when none divides or
// none reads at least a quarter less than the busiest XCD does when the tile
// list -- N-major (tile t is column t / tiles_m) or M-major (row t /
// tiles_n) -- is cut into 8 contiguous ranges.  (Measured on the Llama
// GEMMs: a third less, 384 against 576, is a gain; a tenth less, 640 against
// 704, a loss of 0.14 us.)
inline int xcd_block_grid(int tiles_m, int tiles_n, int bm, int bn_cols, bool n_major) {
  const int G = tiles_m * tiles_n, per = (G + kXcds - 1) / kXcds;
  long cost = 0;
  for (int x = 0; x < kXcds; ++x) {
    const int t0 = x * per, t1 = t0 + per < G ? t0 + per : G;
    if (t0 >= t1) continue;
    const int minor = n_major ? tiles_m : tiles_n;
    const int spans = (t1 - 1) / minor - t0 / minor + 1, within = t1 - t0 < minor ? t1 - t0 : minor;
    const long c = n_major ? (long)within * bm + (long)spans * bn_cols
                           : (long)spans * bm + (long)within * bn_cols;
    if (c > cost) cost = c;
  }
  int best = 0;
  long best_c = 0;
  for (int xm = 1; xm <= kXcds; xm *= 2) {
    const int xn = kXcds / xm;
    if (tiles_m % xm || tiles_n % xn) continue;
    const long c = (long)(tiles_m / xm) * bm + (long)(tiles_n / xn) * bn_cols;
    if (4 * c <= 3 * cost && (best == 0 || c < best_c)) best = xm, best_c = c;
  }
  return best;
}

// Index arithmetic that does not depend on the tile would be hoisted out of
// a tile loop by the compiler and pinned in registers for its whole length;
// passing a value through an empty asm makes it be recomputed per tile
// instead (a few VALU operations against tens of VGPRs).
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Marks a loaded value as used, so the wave waits for its load here.  A
// persistent kernel calls this on everything it loads once (filter
// fragments, bias) before entering its tile loop: the counter of
// outstanding vector-memory operations is in order, so if such a load could
// still be pending inside the loop, the waits the compiler places there for
// it would also drain the next tile's prefetch.
template <class V>
__device__ __forceinline__ void settle(const V &v) {
  asm volatile("" ::"v"(v));
}

// Resident workgroups per CU for `kernel` (launched with `threads` lanes per
// workgroup), times the CU count, rounded down to whole XCD rounds: the
// persistent grid.  Queried once per kernel and device from the runtime
// (register and LDS use decide it); 0 on failure.
template <class K>
int persistent_grid(K kernel, int threads = 256) {
  return cached_per_kernel(reinterpret_cast<const void *>(kernel), [&](int dev) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess)
      return 0;
    return (per_cu > 0 ? per_cu : 1) * cus / kXcds * kXcds;
  });
}

}  // namespace npu
