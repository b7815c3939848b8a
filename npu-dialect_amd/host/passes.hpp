// passes.hpp -- the decisions of NPU-Dialect's pass pipeline, restated
// without MLIR: which ops fuse, how a group is outlined and named, which
// dimension is split across cores and which tile each op gets.  The
// rewriting itself (scf.for nests, extract/insert_slice) is not reproduced:
// on the GPU a group is one launch whose grid is that loop nest.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "cost_model.hpp"

namespace npu {

// FusionPass.cpp:40
constexpr size_t kMaxFusionLength = 6;

// FusionPass.cpp:147-298: greedy vertical fusion.  Anchors in descending
// compute cycles (ties keep block order), forward then backward expansion
// over single-use edges, each step taking the neighbour with the largest
// positive pipelined-cycle benefit.  Only groups of more than one op.
std::vector<std::vector<int32_t>> fusion_groups(const ir::Graph &g, const CostModel &cm);

// FusionPass.cpp:306-359: a (matrix op -> generic) pair tiles the generic by
// its best tile config and fuses the producer into that loop, unless the
// config has a single tile.  Returns false when no tiling happens.
bool tile_and_fuse_decision(const ir::Graph &g, const CostModel &cm, int32_t consumer,
                            TileConfig *config);

struct OutlinedGroup {
  std::vector<int32_t> ops;       // block order
  std::string name;               // fused_<short names>_<idx>
  std::vector<int32_t> inputs;    // external inputs, first-use order
  std::vector<int32_t> outputs;   // used outside, then the last op's results
};

// OutlineFusedGroupsPass.cpp:123-321 over the linalg ops of `scope` (block
// order).  Groups are numbered in the order of their first op.
std::vector<OutlinedGroup> outline_groups(const ir::Graph &g, const CostModel &cm,
                                          const std::vector<int32_t> &scope);
std::string short_op_name(const ir::Graph &g, int32_t op);

struct SpatialDecision {
  int32_t iter_dim = -1, out_dim = -1;
  int64_t dim_size = 0, tile_size = 0, full_iters = 0, peel_size = 0;
  int64_t cost = 0;
  std::vector<std::pair<int32_t, int64_t>> candidates;  // (iter_dim, total cycles)
};
// SpatialTilingPass.cpp:38-168 for one top-level op.
bool spatial_decision(const ir::Graph &g, const CostModel &cm, int32_t op, int64_t cores,
                      SpatialDecision *out);

// TemporalTilingPass.cpp:76-336: spec-driven search, bestTileConfig as the
// fallback; tile sizes in iteration-domain coordinates.  False when the op
// stays untiled (no valid config or a single tile).
bool temporal_decision(const ir::Graph &g, const CostModel &cm, int32_t op, TileConfig *out);

// DMASchedulingPass.cpp:92-147 (npu-barrier-alloc): the schedulable ops of
// a function in program order -- DMA into SRAM, compute (linalg ops and
// memref copies), DMA out of SRAM -- are cut into subgraphs, a new one
// starting at a DMA-in that follows a DMA-out or a compute op; subgraph i
// gets barrier id i % pool and generation i / pool.  Ignored ops keep -1.
enum class SchedKind : int32_t { DmaIn = 0, Compute = 1, DmaOut = 2, Ignore = 3 };
struct BarrierAssignment {
  int64_t subgraph = -1, barrier_id = -1, generation = -1;
};
std::vector<BarrierAssignment> barrier_alloc(const std::vector<SchedKind> &ops, int64_t pool);

}  // namespace npu
