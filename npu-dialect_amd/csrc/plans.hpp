// plans.hpp -- launch plans recorded by the kernel launchers (the per-tile
// work figures of npu_launch_plan, include/npu_amd.h) for the MI355X launch
// model.  Each launcher records one plan per kernel it launches, computed
// from the same template constants and grid it launches with.
#pragma once
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/npu_amd.h"

namespace npu {

// Thread-local plan list of the current entry-point call (defined in abi.hip).
void plans_reset();
void plans_add(const npu_launch_plan &p);

// Resident 256-lane workgroups per CU for `kernel`, from the runtime's
// occupancy calculator (registers and LDS decide it); queried once.
template <class K>
int wg_per_cu(K kernel) {
  static int k = 0;
  if (k == 0) {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, kernel, 256, 0) == hipSuccess) k = v;
  }
  return k;
}

inline npu_launch_plan make_plan(const char *kernel, int grid, int per_cu, int tiles,
                                 int mfma_bits) {
  npu_launch_plan p;
  std::memset(&p, 0, sizeof p);
  std::strncpy(p.kernel, kernel, sizeof p.kernel - 1);
  p.grid = grid;
  p.wg_per_cu = per_cu;
  p.tiles = tiles;
  p.load_phases = 1;
  p.mfma_bits = mfma_bits;
  return p;
}

}  // namespace npu
