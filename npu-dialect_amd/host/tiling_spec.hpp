// tiling_spec.hpp -- per-op split semantics: for each dimension a tile loop
// can split, how every operand is sliced (split, shared, halo, reduce).
// Restates include/npu/Analysis/OperatorTilingSpec.h:42-141 over ir::Graph;
// on the GPU the same rules say which operands a workgroup slices, which it
// replicates and which it loads with a halo.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "ir.hpp"

namespace npu {

enum class SliceKind : int32_t { Split = 0, Shared = 1, Halo = 2, Reduce = 3 };

constexpr uint32_t kNoOutputDim = 0xffffffffu;

struct OperandSliceRule {
  uint32_t operand;
  SliceKind kind;
  uint32_t slice_dim;
  int64_t halo_low = 0;
  int64_t halo_high = 0;
};

struct SplitDimSpec {
  uint32_t output_dim;  // kNoOutputDim for a reduction dimension
  uint32_t iter_dim;
  bool parallel;
  std::vector<OperandSliceRule> input_rules;
  std::vector<OperandSliceRule> output_rules;
  double reuse_ratio = 1.0;
};

struct OperatorTilingSpec {
  std::string op_name;
  std::vector<SplitDimSpec> split_dims;
  int preferred_spatial_dim = -1;
  std::vector<uint32_t> preferred_temporal_dims;
};

OperatorTilingSpec matmul_tiling_spec();
OperatorTilingSpec batch_matmul_tiling_spec();
OperatorTilingSpec conv2d_nchw_tiling_spec(int64_t kh, int64_t kw, int64_t sh, int64_t sw);
// NHWC conv and depthwise conv are not in the reference; their specs follow
// the NCHW one with the dimensions permuted (N, Ho, Wo, F | C).
OperatorTilingSpec conv2d_nhwc_tiling_spec(int64_t kh, int64_t kw);
OperatorTilingSpec depthwise_nhwc_tiling_spec(int64_t kh, int64_t kw);
OperatorTilingSpec elementwise_tiling_spec(unsigned rank);
OperatorTilingSpec generic_tiling_spec(const std::vector<int32_t> &iters, unsigned out_rank);
OperatorTilingSpec transpose_tiling_spec(const std::vector<int64_t> &perm, unsigned rank);

// Registry: the spec of an op, or nullptr.  Matches the reference registry
// (lib/Analysis/OperatorTilingSpec.cpp:518-585) including its caching
// behaviour: the NCHW conv spec is built once per process from the first
// conv it sees (a function-local static, :536).
const OperatorTilingSpec *get_tiling_spec(const ir::Graph &g, int32_t op);
// Forgets the conv spec in force: the next conv asked about builds the next
// one, as the first conv of a fresh npu-opt process does.
void reset_conv_spec();

bool is_reshape_boundary(const ir::Graph &g, int32_t op);

}  // namespace npu
