/*
 * npu_cost.h -- C-ABI of the host-side compiler library (libnpu_host.so):
 * the analytical cost model of lib/Analysis/CostModel.cpp, the per-op split
 * rules of lib/Analysis/OperatorTilingSpec.cpp, and the MI355X target,
 * restated without MLIR over a small SSA graph that the caller builds.
 *
 * A graph is one function body: values (tensor types) and ops in block
 * order.  For linalg ops the operands are `ins` then `outs`, as
 * Operation::getOperands() lists them.  Functions return -1 (and set
 * npu_host_last_error()) on an invalid op or value id.
 */
#ifndef NPU_COST_H
#define NPU_COST_H

#include <stdint.h>

#include "npu_amd.h" /* npu_launch_plan */

#ifdef __cplusplus
extern "C" {
#endif

/* Op kinds (the reference's op vocabulary plus the ops authored here). */
#define NPU_OP_MATMUL 0
#define NPU_OP_BATCH_MATMUL 1
#define NPU_OP_CONV2D_NCHW_FCHW 2
#define NPU_OP_CONV2D_NHWC_FHWC 3
#define NPU_OP_DEPTHWISE_NHWC_HWC 4
#define NPU_OP_GENERIC 5
#define NPU_OP_FILL 6
#define NPU_OP_TRANSPOSE 7
#define NPU_OP_PAD 8
#define NPU_OP_EMPTY 9
#define NPU_OP_CONSTANT 10
#define NPU_OP_RETURN 11
#define NPU_OP_COLLAPSE_SHAPE 12
#define NPU_OP_EXPAND_SHAPE 13
#define NPU_OP_CALL 14
#define NPU_OP_OTHER 15

/* Hardware target: the fields of the reference's HWTarget
 * (include/npu/Analysis/CostModel.h:40-56) and of #npu.target
 * (include/npu/Dialect/NPU/NPUDialect.td:100-113). */
typedef struct npu_hw_target {
  int64_t num_cores;
  int64_t sram_per_core;      /* bytes */
  int64_t dram_bandwidth;     /* GB/s */
  int64_t sram_bandwidth;     /* GB/s */
  int64_t matrix_throughput;  /* MAC / cycle */
  int64_t dsp_throughput;     /* op / cycle */
  int64_t dma_channels;
  int64_t inter_core_sync_cost; /* cycles */
  double clock_ghz;
  int32_t interconnect;       /* 0 NoC, 1 SharedL1, 2 SharedSRAM, 3 DRAMOnly */
  int32_t reserved;
  int64_t noc_bandwidth;      /* GB/s */
  int64_t noc_latency_cycles;
  int64_t shared_l1_size;
} npu_hw_target;

/* The reference's defaults: 6 cores, 2 MiB, 32 GB/s, 4096 MAC/cycle, 1 GHz. */
void npu_hw_target_default(npu_hw_target *t);
/* MI355X per CU for one element width (32, 16 or 8 bits). */
void npu_hw_target_mi355x(npu_hw_target *t, int32_t elem_bits);

typedef struct npu_graph npu_graph;
npu_graph *npu_graph_create(void);
void npu_graph_destroy(npu_graph *g);
/* shaped = 0 for scalars (e.g. the constant a linalg.fill reads). */
int32_t npu_graph_add_value(npu_graph *g, const int64_t *shape, int32_t rank,
                            int32_t bits, int32_t shaped);
/* iters: generic iterator types (0 parallel, 1 reduction); perm: transpose. */
int32_t npu_graph_add_op(npu_graph *g, int32_t kind, const int32_t *operands,
                         int32_t n_operands, const int32_t *results,
                         int32_t n_results, int32_t n_inputs,
                         const int32_t *iters, int32_t n_iters,
                         const int64_t *perm, int32_t n_perm);
int32_t npu_graph_num_ops(const npu_graph *g);

const char *npu_host_last_error(void);

/* ---- level 0 (CostModel.cpp:46-113) ---- */
int64_t npu_cm_op_macs(const npu_graph *g, const npu_hw_target *t, int32_t op);
int64_t npu_cm_compute_cycles(const npu_graph *g, const npu_hw_target *t, int32_t op);
int64_t npu_cm_dma_cycles(const npu_hw_target *t, int64_t bytes);
int64_t npu_cm_tensor_bytes(const int64_t *shape, int32_t rank, int32_t bits);

/* ---- roofline (CostModel.cpp:119-226) ---- */
typedef struct npu_roofline {
  double flops, mem_bytes, arithmetic_intensity, time_sec;
  int32_t is_memory_bound, reserved;
  double peak_attainable, efficiency;
} npu_roofline;
int32_t npu_cm_roofline_raw(const npu_hw_target *t, double flops, double mem_bytes,
                            int32_t matrix, npu_roofline *out);
/* One op (n = 1) or a fused group (external bytes only). */
int32_t npu_cm_roofline(const npu_graph *g, const npu_hw_target *t, const int32_t *ops,
                        int32_t n, npu_roofline *out);

/* ---- level 1 (CostModel.cpp:232-340) ---- */
typedef struct npu_schedule_cost {
  int64_t compute_cycles, dma_cycles, total_cycles, sram_peak_bytes, num_tiles,
      total_dma_bytes;
  int32_t valid, n_tile_sizes;
  int64_t tile_sizes[4];
} npu_schedule_cost;
int32_t npu_cm_matmul_tile(const npu_hw_target *t, int64_t tm, int64_t tn, int64_t tk,
                           int64_t M, int64_t N, int64_t K, int64_t dtype_bytes,
                           int64_t extra_bytes, npu_schedule_cost *out);
int32_t npu_cm_conv2d_tile(const npu_hw_target *t, int64_t tn, int64_t tco, int64_t th,
                           int64_t tw, int64_t N, int64_t Co, int64_t Ho, int64_t Wo,
                           int64_t Ci, int64_t Kh, int64_t Kw, int64_t stride_h,
                           int64_t stride_w, int64_t dtype_bytes,
                           int64_t extra_output_shaped, npu_schedule_cost *out);
/* Writes up to cap candidates, returns how many there are. */
int32_t npu_cm_tile_candidates(int64_t dim, int64_t *out, int32_t cap);
/* The linalg.conv_2d_nchw_fchw tiling spec is built from the first conv it is
 * asked about and then serves every conv (its kernel size sets the halo of the
 * row and column splits), as getTilingSpec's function-local static does for
 * one npu-opt process (OperatorTilingSpec.cpp:531-537).  This forgets it, so
 * the next module's decisions are those of a fresh npu-opt run.  Returns 0. */
int32_t npu_spec_reset(void);

/* ---- level 2 (CostModel.cpp:346-823) ---- */
int32_t npu_cm_best_tile_config(const npu_graph *g, const npu_hw_target *t, int32_t op,
                                npu_schedule_cost *out);
/* Returns 1 if fusing producer into consumer pays, 0 if not; *benefit in cycles. */
int32_t npu_cm_fusion_profitable(const npu_graph *g, const npu_hw_target *t,
                                 int32_t producer, int32_t consumer, int64_t *benefit);
int32_t npu_cm_spatial_split(const npu_graph *g, const npu_hw_target *t, int32_t op,
                             int32_t dim, int64_t chunks, npu_schedule_cost *out);
typedef struct npu_spatial_split_cost {
  int64_t per_core_dma_in_bytes, per_core_compute_cycles, shared_data_bytes,
      split_data_bytes, halo_overhead_bytes;
  int32_t needs_reduce, reserved;
  int64_t total_cycles;
} npu_spatial_split_cost;
/* split_index selects one entry of the op's tiling spec (see npu_spec_*). */
int32_t npu_cm_spatial_split_detailed(const npu_graph *g, const npu_hw_target *t,
                                      int32_t op, int32_t split_index, int64_t chunks,
                                      npu_spatial_split_cost *out);
/* Returns 1 if aligned; *overhead_bytes as the reference computes it. */
int32_t npu_cm_tile_alignment(const npu_graph *g, const npu_hw_target *t, const int32_t *ops,
                              int32_t n, int64_t *overhead_bytes);
/* 0 = retile, 1 = spill. */
int32_t npu_cm_spill_strategy(const npu_hw_target *t, int64_t tile_working_set,
                              int64_t intermediate_bytes);

/* ---- level 3 (CostModel.cpp:829-951) ---- */
typedef struct npu_subgraph_cost {
  int64_t dma_in_cycles, matrix_cycles, dsp_cycles, dma_out_cycles, intermediate_dma,
      pipelined_cycles, unpipelined_cycles, num_ops;
} npu_subgraph_cost;
int32_t npu_cm_subgraph(const npu_graph *g, const npu_hw_target *t, const int32_t *ops,
                        int32_t n, npu_subgraph_cost *out);
int32_t npu_cm_subgraph_fusion_profitable(const npu_graph *g, const npu_hw_target *t,
                                          const int32_t *ops, int32_t n, int64_t *benefit);

/* ---- tiling specs (OperatorTilingSpec.cpp:518-585) ---- */
/* Number of split entries of op's spec (0 if it has none); with index >= 0,
 * fills the entry: output dim (-1 for reduction), iteration dim, parallel. */
int32_t npu_spec_num_splits(const npu_graph *g, int32_t op);
int32_t npu_spec_split(const npu_graph *g, int32_t op, int32_t index, int32_t *output_dim,
                       int32_t *iter_dim, int32_t *parallel);
int32_t npu_spec_preferred_spatial_dim(const npu_graph *g, int32_t op);

/* ---- pass decisions (lib/Transforms) ---- */
/* npu-fusion's greedy groups (FusionPass.cpp:147-298; anchors by descending
 * compute cycles, ties in block order).  Op ids group after group into
 * ops_out, group sizes into sizes_out; returns the number of groups. */
int32_t npu_pass_fusion_groups(const npu_graph *g, const npu_hw_target *t, int32_t *ops_out,
                               int32_t cap_ops, int32_t *sizes_out, int32_t cap_groups);
/* Tile-and-fuse of a (matrix op -> generic) pair (FusionPass.cpp:306-359):
 * 1 and the consumer's tile config if it is tiled, 0 if not. */
int32_t npu_pass_tile_and_fuse(const npu_graph *g, const npu_hw_target *t, int32_t consumer,
                               npu_schedule_cost *out);
/* npu-outline-fused-groups (OutlineFusedGroupsPass.cpp:123-321) over every
 * linalg op; groups numbered by their first op.  Same output convention as
 * npu_pass_fusion_groups. */
int32_t npu_pass_outline_groups(const npu_graph *g, const npu_hw_target *t, int32_t *ops_out,
                                int32_t cap_ops, int32_t *sizes_out, int32_t cap_groups);
/* Name (fused_<ops>_<idx>) and signature of outlined group `index`:
 * external inputs in first-use order, outputs used outside then the last
 * op's results (value ids). */
int32_t npu_pass_outline_group_info(const npu_graph *g, const npu_hw_target *t, int32_t index,
                                    char *name, int32_t name_cap, int32_t *inputs,
                                    int32_t *n_inputs, int32_t *outputs, int32_t *n_outputs,
                                    int32_t cap);
typedef struct npu_spatial_decision {
  int32_t iter_dim, out_dim;
  int64_t dim_size, tile_size, full_iters, peel_size, cost;
  int32_t n_candidates, reserved;
  int32_t cand_iter_dims[8];
  int64_t cand_costs[8];
} npu_spatial_decision;
/* npu-spatial-tiling for one top-level op (SpatialTilingPass.cpp:38-168):
 * 1 if the op is tiled (decision in *out), 0 if it is not a candidate. */
int32_t npu_pass_spatial(const npu_graph *g, const npu_hw_target *t, int32_t op, int64_t cores,
                         npu_spatial_decision *out);
/* npu-temporal-tiling (TemporalTilingPass.cpp:76-336): the number of loops
 * (tile sizes in iteration-domain coordinates, 0 = untiled dim) or 0 if the
 * op stays untiled. */
int32_t npu_pass_temporal(const npu_graph *g, const npu_hw_target *t, int32_t op,
                          npu_schedule_cost *cost, int64_t *tile_sizes, int32_t cap);

/* ---- buffers after tiling: bufferize, SRAM plan, cost record -------------
 * NPUBufferizePass's DMA insertion for one tile loop (BufferizePass.cpp:97-222),
 * NPUSRAMAllocationPass's dual-end plan (SRAMAllocationPass.cpp:127-342) and
 * NPUCostEvaluatePass's per-function record (CostEvaluatePass.cpp:57-168).
 * On MI355X the SRAM is a CU's LDS and the plan a workgroup's LDS layout. */
#define NPU_BUF_INPUT 0        /* copied in, read                          */
#define NPU_BUF_OUTPUT 1       /* copied in, written, copied back          */
#define NPU_BUF_INTERMEDIATE 2 /* lives only in SRAM                       */
typedef struct npu_sram_buffer {
  int32_t value;               /* graph value held, -1 for none           */
  int32_t role;                /* NPU_BUF_*                               */
  int64_t bytes;
  int64_t first_use, last_use; /* program steps                           */
  int32_t in_loop;             /* inside a tile loop: inputs get ping/pong */
  int32_t double_buffered;     /* plan: ping/pong pair                    */
  int64_t addr, addr_pong, prefetch_addr; /* plan: byte offsets, -1 none  */
  int32_t spilled;             /* plan: did not fit, stays in DRAM        */
  int32_t reserved;
} npu_sram_buffer;
typedef struct npu_sram_summary {
  int64_t spilled, prefetched, prefetch_bytes, peak_bytes, free_after;
} npu_sram_summary;
/* Tile loop whose body holds ops[0..n_ops) (block order): one buffer per
 * shaped operand defined outside the body, first-use order; bytes[v] (if
 * bytes and v < n_bytes and bytes[v] > 0) replaces value v's tensor size.
 * Returns the number of buffers (all written to out when cap allows). */
int32_t npu_pass_bufferize(const npu_graph *g, const int32_t *ops, int32_t n_ops,
                           const int64_t *bytes, int32_t n_bytes, npu_sram_buffer *out,
                           int32_t cap);
/* Plans bufs in place for an SRAM of sram_size bytes (summary may be NULL).
 * Buffers are taken in first-use order, ties in array order. */
int32_t npu_pass_sram_allocation(npu_sram_buffer *bufs, int32_t n, int64_t sram_size,
                                 npu_sram_summary *summary);
typedef struct npu_kernel_cost {
  double flops, mem_bytes, arithmetic_intensity, time_sec, efficiency;
  int32_t memory_bound, reserved;
  int64_t dma_in_bytes, dma_out_bytes, matrix_cycles, dsp_cycles;
  int64_t peak_sram_bytes, num_tile_iterations, num_linalg_ops, sram_budget;
} npu_kernel_cost;
/* npu-barrier-alloc (DMASchedulingPass.cpp:92-147): kinds[i] is op i's
 * scheduling class in program order (0 DMA into SRAM, 1 compute, 2 DMA out of
 * SRAM, 3 ignored); subgraph, barrier_id and generation (i % pool, i / pool
 * of its subgraph) are written per op, -1 for ignored ops.  Returns the
 * number of subgraphs, or -1 (pool < 1). */
int32_t npu_pass_barrier_alloc(const int32_t *kinds, int32_t n, int64_t pool, int64_t *subgraph,
                               int64_t *barrier_id, int64_t *generation);

/* The COST_JSON record of a function whose body is ops, its SRAM plan bufs,
 * its tile loops running tile_iterations times. */
int32_t npu_pass_cost_evaluate(const npu_graph *g, const npu_hw_target *t, const int32_t *ops,
                               int32_t n_ops, const npu_sram_buffer *bufs, int32_t n_bufs,
                               int64_t tile_iterations, npu_kernel_cost *out);

/* ---- MI355X launch model ------------------------------------------------
 * Time of one kernel launch from its launch plan (npu_last_launch_plans,
 * npu_amd.h).  The reference's tile pipeline (evaluateConv2dTile /
 * evaluateMatmulTile, CostModel.cpp:232-324: dmaIn + (tiles-1) *
 * max(dmaIn, compute) + compute + dmaOut on one core) is applied per CU, a
 * CU's "tiles" being the work tiles its resident workgroups run.  What a GPU
 * adds to that model: several workgroups per CU overlap one another's load
 * latency; compute is the slowest of the MFMA, LDS and vector-ALU streams;
 * every CU shares one HBM.  Per CU with n tiles and k resident workgroups
 * (each of four waves, one per SIMD), in clocks:
 *   mfma, lds  = macs / MFMA rate, LDS bytes / LDS rate
 *   valu       = a tile's vector instructions per SIMD (valu / 4), issued by
 *                one wave every wave_valu_clk clocks, by a SIMD with k waves
 *                at min(k / wave_valu_clk, valu rate / 4) per clock
 *   xfer       = (load + store bytes) / per-CU L2 rate
 *   serial     = load_phases * latency + xfer + mfma + valu (one wave) + lds
 *                (one tile of one workgroup: its waves' streams in order)
 *   throughput = n * max(lds, mfma + valu (k waves per SIMD), xfer)
 *   rounds     = ceil(n / k) * serial       (a workgroup runs its tiles in turn)
 *   setup      = latency + k * setup bytes / burst rate  (if it has setup data:
 *                the k workgroups of a CU fetch theirs at once), then the
 *                set-up vector instructions per SIMD, one wave at a time
 *                (setup valu / 4 * wave_valu_clk)
 *   cu         = setup + max(throughput, rounds)
 *   time       = max(cu / clock, HBM bytes / HBM bandwidth)
 * The machine constants come from the MI355X data sheet (CUs, MFMA rates)
 * and from npu_calibrate (clock under MFMA load, latency, copy bandwidth, L2,
 * LDS and burst rates, vector issue rates, launch cost). */
typedef struct npu_gpu_params {
  int32_t cus;
  int32_t reserved;
  double clock_ghz;
  double hbm_gbs;               /* achievable HBM bandwidth (device copy)      */
  double l2_bytes_per_clk_cu;   /* L2 -> CU read rate                          */
  double lds_bytes_per_clk_cu;  /* conflict-free 16-byte LDS reads             */
  double valu_instr_per_clk_cu; /* wave vector instructions, four waves/SIMD  */
  double mfma_macs_per_clk_cu[3]; /* f32, bf16, i8 (dense)                    */
  double mem_latency_us;        /* dependent global load with every CU loading */
  double launch_us;             /* per kernel in a captured graph of launches
                                   (an empty kernel's cost, npu_calibrate)    */
  double wave_valu_clk;         /* clocks between one wave's vector
                                   instructions                               */
  double burst_bytes_per_clk_cu; /* one buffer read by every CU at once       */
} npu_gpu_params;
void npu_gpu_params_mi355x(npu_gpu_params *p);

#define NPU_BOUND_HBM 0
#define NPU_BOUND_MFMA 1
#define NPU_BOUND_LDS 2
#define NPU_BOUND_VALU 3
#define NPU_BOUND_L2 4
#define NPU_BOUND_LATENCY 5
typedef struct npu_launch_cost {
  double time_us;      /* predicted kernel duration                          */
  double hbm_us;       /* HBM bytes at the achievable bandwidth               */
  double cu_us;        /* per-CU pipeline time                                */
  double tile_compute_us, tile_xfer_us, tile_serial_us; /* one tile           */
  double tiles_per_cu;
  int32_t bound;       /* NPU_BOUND_*                                         */
  int32_t reserved;
} npu_launch_cost;
/* 0 on success, -1 on an invalid plan (message in npu_host_last_error). */
int32_t npu_cm_predict_launch(const npu_launch_plan *plan, const npu_gpu_params *gpu,
                              npu_launch_cost *out);

#ifdef __cplusplus
}
#endif
#endif /* NPU_COST_H */
