// launch_model.cpp -- the MI355X launch model (npu_cm_predict_launch,
// include/npu_cost.h): the reference's per-core tile pipeline
// (lib/Analysis/CostModel.cpp:232-324) applied per CU, with what a GPU adds
// (resident workgroups overlapping latency, MFMA/LDS/VALU streams, one shared
// HBM).
#include <algorithm>
#include <cmath>

#include "../../include/npu_cost.h"

namespace npu {

// Machine constants.  Data sheet: 256 CUs at 2.4 GHz; dense MFMA per CU per
// clock 128 f32, 2048 bf16 and 4096 i8 multiply-adds (157.3 / 2516.6 /
// 5033.2 T op/s).  Measured on an MI355X with npu_calibrate
// (calib/calibrate.hip): 4.2 TB/s for a 1 GiB device copy, 52 bytes/clock/CU
// read from L2, 1.2 us dependent-load latency with every CU loading (0.31 us
// idle; 0.13 us from L2), 204 bytes/clock/CU of conflict-free ds_read_b128
// (four waves, 20 clocks per wave instruction), one wave64 vector-ALU
// instruction per SIMD every 2 clocks (2 per CU per clock, four waves per
// SIMD), 1.58 us per kernel in a captured graph of empty kernels.
void gpu_params_mi355x(npu_gpu_params *p) {
  p->cus = 256;
  p->reserved = 0;
  p->clock_ghz = 2.4;
  p->hbm_gbs = 4312.0;
  p->l2_bytes_per_clk_cu = 51.0;
  p->lds_bytes_per_clk_cu = 204.0;
  p->valu_instr_per_clk_cu = 2.0;
  p->mfma_macs_per_clk_cu[0] = 128.0;
  p->mfma_macs_per_clk_cu[1] = 2048.0;
  p->mfma_macs_per_clk_cu[2] = 4096.0;
  p->mem_latency_us = 1.2;
  p->launch_us = 1.58;
}

bool predict_launch(const npu_launch_plan &pl, const npu_gpu_params &g, npu_launch_cost *out) {
  if (pl.grid <= 0 || pl.tiles <= 0 || g.cus <= 0 || g.clock_ghz <= 0) return false;
  const int mi = pl.mfma_bits >= 32 ? 0 : (pl.mfma_bits >= 16 ? 1 : 2);
  const double clk_per_us = g.clock_ghz * 1e3;
  // compute streams of one tile, in clocks of one CU
  const double c_mfma = pl.tile_macs / g.mfma_macs_per_clk_cu[mi];
  const double c_lds = pl.tile_lds_bytes / g.lds_bytes_per_clk_cu;
  const double c_valu = pl.tile_valu / g.valu_instr_per_clk_cu;
  const double c_comp = std::max(c_lds, c_mfma + c_valu);
  const double c_xfer = (pl.tile_load_bytes + pl.tile_store_bytes) / g.l2_bytes_per_clk_cu;
  const double c_lat = pl.load_phases * g.mem_latency_us * clk_per_us;
  const double c_serial = c_lat + c_xfer + c_comp;
  // tiles per CU (the busiest CU) and resident workgroups overlapping them
  const double tiles_cu = std::ceil((double)pl.tiles / g.cus);
  const double wgs_cu = std::ceil((double)pl.grid / g.cus);
  const double k = std::max(1.0, std::min((double)std::max(pl.wg_per_cu, 1), wgs_cu));
  const double setup = g.mem_latency_us * clk_per_us + pl.wg_setup_bytes / g.l2_bytes_per_clk_cu;
  const double c_thru = tiles_cu * std::max(c_comp, c_xfer);
  const double c_latb = tiles_cu * c_serial / k;
  const double cu = setup + std::max(c_thru, c_latb);
  const double hbm_us = pl.hbm_bytes / (g.hbm_gbs * 1e3);
  out->hbm_us = hbm_us;
  out->cu_us = cu / clk_per_us;
  out->tile_compute_us = c_comp / clk_per_us;
  out->tile_xfer_us = c_xfer / clk_per_us;
  out->tile_serial_us = c_serial / clk_per_us;
  out->tiles_per_cu = tiles_cu;
  out->time_us = std::max(out->cu_us, hbm_us);
  if (hbm_us >= out->cu_us)
    out->bound = NPU_BOUND_HBM;
  else if (c_latb > c_thru)
    out->bound = NPU_BOUND_LATENCY;
  else if (c_xfer >= c_comp)
    out->bound = NPU_BOUND_L2;
  else if (c_lds >= c_mfma + c_valu)
    out->bound = NPU_BOUND_LDS;
  else if (c_mfma >= c_valu)
    out->bound = NPU_BOUND_MFMA;
  else
    out->bound = NPU_BOUND_VALU;
  out->reserved = 0;
  return true;
}

}  // namespace npu
