// memory_plan.hpp -- the buffer decisions made after tiling, MLIR-free:
//   * NPUBufferizePass's DMA insertion for a tile loop
//     (lib/Transforms/BufferizePass.cpp:97-222): every memref defined outside
//     the loop and used inside it gets an SRAM buffer and a DRAM->SRAM copy
//     at the loop start; the ones written inside get an SRAM->DRAM copy
//     before the yield;
//   * NPUSRAMAllocationPass's dual-end plan
//     (lib/Transforms/SRAMAllocationPass.cpp:127-342): liveness by program
//     step, inputs from the low end, outputs from the high end, intermediates
//     in the middle, 64-byte alignment, ping/pong for inputs inside a tile
//     loop, spill to DRAM when nothing fits, weight prefetch into what is
//     left;
//   * NPUCostEvaluatePass's per-function record (CostEvaluatePass.cpp:57-168).
// On the GPU the SRAM is a CU's LDS (160 KiB) and the plan is a workgroup's
// LDS layout.
#pragma once
#include <cstdint>
#include <vector>

#include "cost_model.hpp"
#include "ir.hpp"

namespace npu {

enum class BufRole : int32_t { Input = 0, Output = 1, Intermediate = 2 };

struct SramBuffer {
  // description
  int32_t value = -1;        // graph value held (-1: none)
  int64_t bytes = 0;
  BufRole role = BufRole::Intermediate;
  int64_t first_use = 0, last_use = 0;  // program steps
  bool in_loop = true;       // inside a tile loop: an input gets ping/pong
  // plan
  int64_t addr = -1, addr_pong = -1, prefetch_addr = -1;
  bool double_buffered = false, spilled = false;
};

// SRAMAllocationPass.cpp:127-162: a bump allocator from both ends.
struct DualEndAllocator {
  int64_t size, low = 0, high;
  explicit DualEndAllocator(int64_t s) : size(s), high(s) {}
  static int64_t align(int64_t b) { return (b + 63) & ~int64_t(63); }
  int64_t alloc_low(int64_t b);
  int64_t alloc_high(int64_t b);
  int64_t alloc_middle(int64_t b) { return alloc_low(b); }
  void free_low(int64_t b);
  int64_t free_bytes() const { return high - low; }
};

struct SramPlanSummary {
  int64_t spilled = 0, prefetched = 0, prefetch_bytes = 0, peak_bytes = 0, free_after = 0;
};

// Phases 1-4 of the pass over `bufs` (in place).  Buffers are visited in
// first-use order; equal first uses keep their given order (the reference
// sorts with an unstable std::sort there, so its order among ties is
// unspecified).
SramPlanSummary plan_sram(std::vector<SramBuffer> &bufs, int64_t sram_size);

// DMA insertion for the tile loop whose body holds `ops` (block order), e.g.
// a fused group after tile-and-fuse.  Every shaped operand defined outside
// the body (not an arith.constant) becomes one SRAM buffer, in first-use
// order; operands in a linalg op's `outs` are written (copied back).  In
// program steps the loop body is: alloc_sram and dma_copy per buffer, the
// ops, then the copies back.  `bytes` (optional, indexed by value) replaces
// a value's full tensor size, e.g. by its tile slice.
std::vector<SramBuffer> bufferize_loop(const ir::Graph &g, const std::vector<int32_t> &ops,
                                       const std::vector<int64_t> *bytes = nullptr);

// CostEvaluatePass.cpp:57-168 for a function whose body is `ops`, its tile
// loops running `tile_iterations` times, its SRAM plan `bufs`.
struct KernelCost {
  double flops = 0, mem_bytes = 0, arithmetic_intensity = 0, time_sec = 0, efficiency = 0;
  bool memory_bound = true;
  int64_t dma_in_bytes = 0, dma_out_bytes = 0, matrix_cycles = 0, dsp_cycles = 0;
  int64_t peak_sram_bytes = 0, num_tile_iterations = 1, num_linalg_ops = 0, sram_budget = 0;
};
KernelCost cost_evaluate(const ir::Graph &g, const CostModel &cm, const std::vector<int32_t> &ops,
                         const std::vector<SramBuffer> &bufs, int64_t tile_iterations);

}  // namespace npu
