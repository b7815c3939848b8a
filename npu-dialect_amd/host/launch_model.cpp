// launch_model.cpp -- the MI355X launch model (npu_cm_predict_launch,
// include/npu_cost.h): the reference's per-core tile pipeline
// (lib/Analysis/CostModel.cpp:232-324) applied per CU, with what a GPU adds
// (resident workgroups overlapping latency, MFMA/LDS/VALU streams, one shared
// HBM).
#include <algorithm>
#include <cmath>

#include "../../include/npu_cost.h"

namespace npu {

// Machine constants.  Data sheet: 256 CUs; dense MFMA per CU per clock 128
// f32, 2048 bf16 and 4096 i8 multiply-adds (157.3 / 2516.6 / 5033.2 T op/s
// at 2.4 GHz).  Measured on an MI355X with npu_calibrate
// (calib/calibrate.hip): a 2.37 GHz shader clock with every CU running
// MFMAs; 4.2 TB/s for a 1 GiB device copy; 51 bytes/clock/CU read from L2;
// 34 bytes/clock/CU when every CU reads the same 144 KiB at once (a
// persistent kernel's filter fetch); 1.2 us dependent-load latency with
// every CU loading (0.31 us idle, 0.13 us from L2); 204 bytes/clock/CU of
// conflict-free ds_read_b128 (four waves, 20 clocks per wave instruction);
// one vector instruction per SIMD every 2 clocks with four waves per SIMD,
// every 8 clocks from a single wave; 1.58 us per kernel in a captured graph
// of empty kernels.
void gpu_params_mi355x(npu_gpu_params *p) {
  p->cus = 256;
  p->reserved = 0;
  p->clock_ghz = 2.37;
  p->hbm_gbs = 4210.0;
  p->l2_bytes_per_clk_cu = 51.0;
  p->lds_bytes_per_clk_cu = 204.0;
  p->valu_instr_per_clk_cu = 2.0;
  p->mfma_macs_per_clk_cu[0] = 128.0;
  p->mfma_macs_per_clk_cu[1] = 2048.0;
  p->mfma_macs_per_clk_cu[2] = 4096.0;
  p->mem_latency_us = 1.2;
  p->launch_us = 1.58;
  p->wave_valu_clk = 8.0;
  p->burst_bytes_per_clk_cu = 34.4;
}

// The formula is written out in include/npu_cost.h.
bool predict_launch(const npu_launch_plan &pl, const npu_gpu_params &g, npu_launch_cost *out) {
  if (pl.grid <= 0 || pl.tiles <= 0 || g.cus <= 0 || g.clock_ghz <= 0 || g.wave_valu_clk <= 0 ||
      g.valu_instr_per_clk_cu <= 0 || g.burst_bytes_per_clk_cu <= 0)
    return false;
  const int mi = pl.mfma_bits >= 32 ? 0 : (pl.mfma_bits >= 16 ? 1 : 2);
  const double clk_per_us = g.clock_ghz * 1e3;
  // tiles per CU (the busiest CU) and resident workgroups sharing it
  const double tiles_cu = std::ceil((double)pl.tiles / g.cus);
  const double wgs_cu = std::ceil((double)pl.grid / g.cus);
  const double k = std::max(1.0, std::min((double)std::max(pl.wg_per_cu, 1), wgs_cu));
  // streams of one tile, in clocks of one CU
  const double c_mfma = pl.tile_macs / g.mfma_macs_per_clk_cu[mi];
  const double c_lds = pl.tile_lds_bytes / g.lds_bytes_per_clk_cu;
  const double valu_simd = pl.tile_valu / 4.0;
  const double c_valu_wave = valu_simd * g.wave_valu_clk;
  const double c_valu_k = valu_simd / std::min(k / g.wave_valu_clk, g.valu_instr_per_clk_cu / 4.0);
  const double c_xfer = (pl.tile_load_bytes + pl.tile_store_bytes) / g.l2_bytes_per_clk_cu;
  const double c_lat = pl.load_phases * g.mem_latency_us * clk_per_us;
  const double c_comp = std::max(c_lds, c_mfma + c_valu_k);
  const double c_serial = c_lat + c_xfer + c_mfma + c_valu_wave + c_lds;
  const double c_thru = tiles_cu * std::max(c_comp, c_xfer);
  const double c_rounds = std::ceil(tiles_cu / k) * c_serial;
  const double setup = (pl.wg_setup_bytes > 0
                            ? g.mem_latency_us * clk_per_us + k * pl.wg_setup_bytes / g.burst_bytes_per_clk_cu
                            : 0.0) +
                       pl.wg_setup_valu / 4.0 * g.wave_valu_clk;
  const double cu = setup + std::max(c_thru, c_rounds);
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
  else if (c_rounds > c_thru)
    out->bound = NPU_BOUND_LATENCY;
  else if (c_xfer >= c_comp)
    out->bound = NPU_BOUND_L2;
  else if (c_lds >= c_mfma + c_valu_k)
    out->bound = NPU_BOUND_LDS;
  else if (c_mfma >= c_valu_k)
    out->bound = NPU_BOUND_MFMA;
  else
    out->bound = NPU_BOUND_VALU;
  out->reserved = 0;
  return true;
}

}  // namespace npu
