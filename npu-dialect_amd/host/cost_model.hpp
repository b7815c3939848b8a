// cost_model.hpp -- the analytical cost model shared by the decision passes
// (restatement of include/npu/Analysis/CostModel.h:33-272 over ir::Graph),
// plus its MI355X target.
#pragma once
#include <cstdint>
#include <vector>

#include "ir.hpp"
#include "tiling_spec.hpp"

namespace npu {

enum class Interconnect : int32_t { NoC = 0, SharedL1 = 1, SharedSRAM = 2, DRAMOnly = 3 };

// Hardware description.  The defaults are the reference's fictional NPU
// (CostModel.h:40-56): 6 cores, 2 MiB SRAM each, 32 GB/s, 4096 MAC/cycle
// matrix, 256 op/cycle DSP, 1 GHz.
struct HWTarget {
  int64_t num_cores = 6;
  int64_t sram_per_core = 2 * 1024 * 1024;
  int64_t dram_bandwidth = 32;       // GB/s
  int64_t sram_bandwidth = 256;      // GB/s
  int64_t matrix_throughput = 4096;  // MAC/cycle
  int64_t dsp_throughput = 256;      // op/cycle
  int64_t dma_channels = 2;
  int64_t inter_core_sync_cost = 100;  // cycles
  double clock_ghz = 1.0;
  Interconnect interconnect = Interconnect::NoC;
  int64_t noc_bandwidth = 128;       // GB/s
  int64_t noc_latency_cycles = 10;
  int64_t shared_l1_size = 0;

  double bytes_per_cycle() const { return (double)dram_bandwidth / clock_ghz; }
  double noc_bytes_per_cycle() const { return (double)noc_bandwidth / clock_ghz; }
  int64_t inter_core_transfer_cycles(int64_t bytes) const;
};

// The MI355X seen through the same parameters, for one element type
// (32 = f32, 16 = bf16, 8 = i8): a "core" is a CU (256 of them, 2.4 GHz),
// its SRAM the 160 KiB LDS, the matrix engine the CU's MFMA rate for that
// type (per CU per cycle: 128 MAC f32, 2048 MAC bf16, 4096 MAC i8), the DSP
// the CU's 64 FP32 lanes, DRAM the CU's share of 8 TB/s HBM3E (31 GB/s when
// all 256 CUs stream), inter-CU data through the shared L2 (SharedSRAM).
HWTarget mi355x_target(int32_t elem_bits);

struct ScheduleCost {
  int64_t compute_cycles = 0;
  int64_t dma_cycles = 0;
  int64_t total_cycles = 0;
  int64_t sram_peak_bytes = 0;
  int64_t num_tiles = 0;
  int64_t total_dma_bytes = 0;
  bool valid() const;
};

struct RooflineCost {
  double flops = 0, mem_bytes = 0, arithmetic_intensity = 0, time_sec = 0;
  bool memory_bound = true;
  double peak_attainable = 0, efficiency = 0;
};

struct FusionDecision {
  bool fuse = false;
  int64_t benefit_cycles = 0;
};

struct TileConfig {
  std::vector<int64_t> tile_sizes;
  ScheduleCost cost;
};

struct SpatialSplitCost {
  int64_t per_core_dma_in_bytes = 0;
  int64_t per_core_compute_cycles = 0;
  int64_t shared_data_bytes = 0;
  int64_t split_data_bytes = 0;
  int64_t halo_overhead_bytes = 0;
  bool needs_reduce = false;
  int64_t total_cycles = 0;
};

struct TileAlignment {
  bool aligned = false;
  int64_t overhead_bytes = 0;
};

struct SubgraphCost {
  int64_t dma_in_cycles = 0, matrix_cycles = 0, dsp_cycles = 0, dma_out_cycles = 0;
  int64_t intermediate_dma = 0, pipelined_cycles = 0, unpipelined_cycles = 0, num_ops = 0;
};

enum class SpillStrategy : int32_t { Retile = 0, Spill = 1 };

class CostModel {
 public:
  CostModel(const ir::Graph &g, const HWTarget &t) : g_(g), t_(t) {}
  const HWTarget &target() const { return t_; }

  // Level 0 (CostModel.cpp:46-113)
  int64_t op_macs(int32_t op) const;
  bool is_matrix_op(int32_t op) const;
  int64_t compute_cycles(int32_t op) const;
  int64_t dma_cycles(int64_t bytes) const;
  static int64_t tensor_bytes(const ir::Type &t);

  // Roofline (CostModel.cpp:119-226)
  RooflineCost roofline_raw(double flops, double mem_bytes, bool matrix) const;
  RooflineCost roofline(int32_t op) const;
  RooflineCost roofline(const std::vector<int32_t> &ops) const;

  // Level 1 (CostModel.cpp:232-340)
  ScheduleCost matmul_tile(int64_t tm, int64_t tn, int64_t tk, int64_t M, int64_t N, int64_t K,
                           int64_t dtype_bytes, int64_t extra_bytes = 0) const;
  ScheduleCost conv2d_tile(int64_t tn, int64_t tco, int64_t th, int64_t tw, int64_t N,
                           int64_t Co, int64_t Ho, int64_t Wo, int64_t Ci, int64_t Kh, int64_t Kw,
                           const std::vector<int64_t> &stride, int64_t dtype_bytes,
                           int64_t extra_output_shaped = 0) const;
  static std::vector<int64_t> tile_candidates(int64_t dim);

  // Level 2 (CostModel.cpp:346-823)
  TileConfig best_tile_config(int32_t op) const;
  FusionDecision fusion_profitable(int32_t producer, int32_t consumer) const;
  ScheduleCost spatial_split(int32_t op, unsigned dim, int64_t chunks) const;
  SpatialSplitCost spatial_split_detailed(int32_t op, const SplitDimSpec &spec,
                                          int64_t chunks) const;
  TileAlignment tile_alignment(const std::vector<int32_t> &ops) const;
  SpillStrategy spill_strategy(int64_t tile_working_set, int64_t intermediate_bytes) const;

  // Level 3 (CostModel.cpp:829-951)
  SubgraphCost subgraph(const std::vector<int32_t> &ops) const;
  FusionDecision subgraph_fusion_profitable(const std::vector<int32_t> &ops) const;

 private:
  const ir::Graph &g_;
  HWTarget t_;
};

}  // namespace npu
