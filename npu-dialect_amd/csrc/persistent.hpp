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
