// plans.hpp -- launch plans recorded by the kernel launchers (the per-tile
// work figures of npu_launch_plan, include/npu_amd.h) for the MI355X launch
// model.  Each launcher records one plan per kernel it launches, computed
// from the same template constants and grid it launches with.
#pragma once
#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <mutex>
#include <utility>

#include "../../include/npu_amd.h"

namespace npu {

// Thread-local plan list of the current entry-point call (defined in abi.hip).
void plans_reset();
void plans_add(const npu_launch_plan &p);
// Sets the calling thread's npu_last_error() message (defined in abi.hip).
void set_last_error(const char *msg);
// The typed entry points' descriptor check (rank, dtype, row-major
// contiguity, alignment, element limit); on failure the message is the
// thread's last error.
npu_status memref_check(const npu_memref *m, const char *name, int32_t rank, int32_t dtype);

// Per-kernel, per-device launch facts cached by kernel address (kernels of
// one signature share a function type, so the type cannot be the key).
// Returns the cached value of (kernel, current device), computing it with
// `compute(device)` the first time; 0 if the device cannot be queried or
// `compute` reports 0.
template <class F>
int cached_per_kernel(const void *kernel, F compute) {
  static std::mutex mu;
  static std::map<std::pair<const void *, int>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find({kernel, dev});
  if (it != cache.end()) return it->second;
  const int v = compute(dev);
  if (v > 0) cache[{kernel, dev}] = v;
  return v;
}

// Resident four-wave units per CU for `kernel` launched with `threads`
// lanes per workgroup (resident workgroups x threads / 256), from the
// runtime's occupancy calculator (registers and LDS decide it): the waves
// each SIMD holds.
template <class K>
int wg_per_cu(K kernel, int threads = 256) {
  return cached_per_kernel(reinterpret_cast<const void *>(kernel), [&](int) {
    int v = 0;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, kernel, threads, 0) == hipSuccess
               ? v * threads / 256
               : 0;
  });
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
  p.unit_waves = 4;
  return p;
}

}  // namespace npu
