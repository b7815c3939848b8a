// tiling_spec.cpp -- split rules per op kind (the tables of
// lib/Analysis/OperatorTilingSpec.cpp:21-413, kept alike because decisions
// made from them must agree with the reference's).
#include "tiling_spec.hpp"

#include <map>
#include <memory>
#include <mutex>

namespace npu {

using ir::OpKind;

namespace {

SplitDimSpec split(uint32_t out_dim, uint32_t iter_dim, bool parallel,
                   std::vector<OperandSliceRule> in, std::vector<OperandSliceRule> out,
                   double reuse) {
  SplitDimSpec s;
  s.output_dim = out_dim;
  s.iter_dim = iter_dim;
  s.parallel = parallel;
  s.input_rules = std::move(in);
  s.output_rules = std::move(out);
  s.reuse_ratio = reuse;
  return s;
}

constexpr SliceKind S = SliceKind::Split, SH = SliceKind::Shared, HA = SliceKind::Halo,
                    RE = SliceKind::Reduce;

}  // namespace

// C[M,N] = A[M,K] B[K,N]: split M (B shared), split N (A shared), split K (reduce).
OperatorTilingSpec matmul_tiling_spec() {
  OperatorTilingSpec spec;
  spec.op_name = "linalg.matmul";
  spec.split_dims.push_back(split(0, 0, true, {{0, S, 0}, {1, SH, 0}}, {{0, S, 0}}, 2.0));
  spec.split_dims.push_back(split(1, 1, true, {{0, SH, 0}, {1, S, 1}}, {{0, S, 1}}, 2.0));
  spec.split_dims.push_back(
      split(kNoOutputDim, 2, false, {{0, S, 1}, {1, S, 0}}, {{0, RE, 0}}, 1.0));
  spec.preferred_spatial_dim = 0;
  spec.preferred_temporal_dims = {0, 1, 2};
  return spec;
}

// C[B,M,N] = A[B,M,K] B[B,K,N].
OperatorTilingSpec batch_matmul_tiling_spec() {
  OperatorTilingSpec spec;
  spec.op_name = "linalg.batch_matmul";
  spec.split_dims.push_back(split(0, 0, true, {{0, S, 0}, {1, S, 0}}, {{0, S, 0}}, 1.0));
  spec.split_dims.push_back(split(1, 1, true, {{0, S, 1}, {1, SH, 0}}, {{0, S, 1}}, 2.0));
  spec.split_dims.push_back(split(2, 2, true, {{0, SH, 0}, {1, S, 2}}, {{0, S, 2}}, 2.0));
  spec.split_dims.push_back(
      split(kNoOutputDim, 3, false, {{0, S, 2}, {1, S, 1}}, {{0, RE, 0}}, 1.0));
  spec.preferred_spatial_dim = 1;
  spec.preferred_temporal_dims = {0, 1, 2, 3};
  return spec;
}

// O[N,F,Ho,Wo] over I[N,C,Hi,Wi], K[F,C,Kh,Kw]; Ho / Wo splits need a halo of
// Kh-1 / Kw-1 input rows / columns.
OperatorTilingSpec conv2d_nchw_tiling_spec(int64_t kh, int64_t kw, int64_t, int64_t) {
  OperatorTilingSpec spec;
  spec.op_name = "linalg.conv_2d_nchw_fchw";
  spec.split_dims.push_back(split(0, 0, true, {{0, S, 0}, {1, SH, 0}}, {{0, S, 0}}, 3.0));
  spec.split_dims.push_back(split(1, 1, true, {{0, SH, 0}, {1, S, 0}}, {{0, S, 1}}, 2.0));
  spec.split_dims.push_back(
      split(2, 2, true, {{0, HA, 2, 0, kh - 1}, {1, SH, 0}}, {{0, S, 2}}, 1.5));
  spec.split_dims.push_back(
      split(3, 3, true, {{0, HA, 3, 0, kw - 1}, {1, SH, 0}}, {{0, S, 3}}, 1.5));
  spec.split_dims.push_back(
      split(kNoOutputDim, 4, false, {{0, S, 1}, {1, S, 1}}, {{0, RE, 0}}, 1.0));
  spec.preferred_spatial_dim = 1;
  spec.preferred_temporal_dims = {2, 3, 1};
  return spec;
}

// O[N,Ho,Wo,F] over I[N,Hi,Wi,C], K[F,Kh,Kw,C].
OperatorTilingSpec conv2d_nhwc_tiling_spec(int64_t kh, int64_t kw) {
  OperatorTilingSpec spec;
  spec.op_name = "linalg.conv_2d_nhwc_fhwc";
  spec.split_dims.push_back(split(0, 0, true, {{0, S, 0}, {1, SH, 0}}, {{0, S, 0}}, 3.0));
  spec.split_dims.push_back(
      split(1, 1, true, {{0, HA, 1, 0, kh - 1}, {1, SH, 0}}, {{0, S, 1}}, 1.5));
  spec.split_dims.push_back(
      split(2, 2, true, {{0, HA, 2, 0, kw - 1}, {1, SH, 0}}, {{0, S, 2}}, 1.5));
  spec.split_dims.push_back(split(3, 3, true, {{0, SH, 0}, {1, S, 0}}, {{0, S, 3}}, 2.0));
  spec.split_dims.push_back(
      split(kNoOutputDim, 4, false, {{0, S, 3}, {1, S, 3}}, {{0, RE, 0}}, 1.0));
  spec.preferred_spatial_dim = 3;
  spec.preferred_temporal_dims = {1, 2, 3};
  return spec;
}

// O[N,Ho,Wo,C] over I[N,Hi,Wi,C], K[Kh,Kw,C]: channels split both operands.
OperatorTilingSpec depthwise_nhwc_tiling_spec(int64_t kh, int64_t kw) {
  OperatorTilingSpec spec;
  spec.op_name = "linalg.depthwise_conv_2d_nhwc_hwc";
  spec.split_dims.push_back(split(0, 0, true, {{0, S, 0}, {1, SH, 0}}, {{0, S, 0}}, 3.0));
  spec.split_dims.push_back(
      split(1, 1, true, {{0, HA, 1, 0, kh - 1}, {1, SH, 0}}, {{0, S, 1}}, 1.5));
  spec.split_dims.push_back(
      split(2, 2, true, {{0, HA, 2, 0, kw - 1}, {1, SH, 0}}, {{0, S, 2}}, 1.5));
  spec.split_dims.push_back(split(3, 3, true, {{0, S, 3}, {1, S, 2}}, {{0, S, 3}}, 1.0));
  spec.preferred_spatial_dim = 3;
  spec.preferred_temporal_dims = {1, 2, 3};
  return spec;
}

OperatorTilingSpec elementwise_tiling_spec(unsigned rank) {
  OperatorTilingSpec spec;
  spec.op_name = "linalg.generic (elementwise)";
  for (unsigned d = 0; d < rank; ++d)
    spec.split_dims.push_back(split(d, d, true, {{0, S, d}}, {{0, S, d}}, 1.0));
  spec.preferred_spatial_dim = 0;
  spec.preferred_temporal_dims = {0};
  return spec;
}

// From iterator types: parallel dims map to output dims in order; reduction
// dims split the input and make the output a partial sum.
OperatorTilingSpec generic_tiling_spec(const std::vector<int32_t> &iters, unsigned out_rank) {
  OperatorTilingSpec spec;
  unsigned npar = 0, nred = 0;
  for (int32_t t : iters) (t == 0 ? npar : nred)++;
  spec.op_name = nred == 0 ? "linalg.generic (elementwise)"
                 : npar > 0 ? "linalg.generic (mixed par/red)"
                            : "linalg.generic (full reduction)";
  unsigned out_idx = 0;
  for (unsigned d = 0; d < iters.size(); ++d) {
    const bool par = iters[d] == 0;
    if (par && out_idx < out_rank) {
      spec.split_dims.push_back(split(out_idx, d, true, {{0, S, out_idx}}, {{0, S, out_idx}}, 1.0));
      ++out_idx;
    } else {
      spec.split_dims.push_back(split(kNoOutputDim, d, par, {{0, S, d < out_rank ? d : 0u}},
                                      {{0, RE, 0}}, 1.0));
    }
  }
  for (unsigned d = 0; d < iters.size(); ++d)
    if (iters[d] == 0) {
      if (spec.preferred_spatial_dim == -1) spec.preferred_spatial_dim = (int)d;
      spec.preferred_temporal_dims.push_back(d);
    }
  for (unsigned d = 0; d < iters.size(); ++d)
    if (iters[d] != 0) spec.preferred_temporal_dims.push_back(d);
  return spec;
}

OperatorTilingSpec transpose_tiling_spec(const std::vector<int64_t> &perm, unsigned rank) {
  OperatorTilingSpec spec;
  spec.op_name = "linalg.transpose";
  for (unsigned d = 0; d < rank; ++d)
    spec.split_dims.push_back(
        split(d, d, true, {{0, S, (uint32_t)perm[d]}}, {{0, S, d}}, 1.0));
  spec.preferred_spatial_dim = 0;
  return spec;
}

bool is_reshape_boundary(const ir::Graph &g, int32_t op) {
  const OpKind k = g.ops[op].kind;
  return k == OpKind::CollapseShape || k == OpKind::ExpandShape;
}

namespace {
// The conv spec in force and every one built so far (a spec handed out stays
// valid after a reset).
std::mutex conv_mu;
std::vector<std::unique_ptr<OperatorTilingSpec>> conv_specs;
const OperatorTilingSpec *conv_current = nullptr;
}  // namespace

void reset_conv_spec() {
  std::lock_guard<std::mutex> lock(conv_mu);
  conv_current = nullptr;
}

const OperatorTilingSpec *get_tiling_spec(const ir::Graph &g, int32_t opi) {
  static const OperatorTilingSpec mm = matmul_tiling_spec();
  static const OperatorTilingSpec bmm = batch_matmul_tiling_spec();
  static std::mutex mu;
  static std::map<std::vector<int64_t>, OperatorTilingSpec> cache;
  const ir::Op &op = g.ops[opi];
  switch (op.kind) {
    case OpKind::Matmul:
      return &mm;
    case OpKind::BatchMatmul:
      return &bmm;
    case OpKind::Conv2dNchwFchw: {
      // Built from the first conv asked about, strides taken as 1, and kept
      // for every later conv until reset_conv_spec (the reference's
      // function-local static: one spec per npu-opt process).
      const auto &ft = g.type(op.operands[1]).shape;
      std::lock_guard<std::mutex> lock(conv_mu);
      if (!conv_current) {
        conv_specs.push_back(std::make_unique<OperatorTilingSpec>(
            conv2d_nchw_tiling_spec(ft[2], ft[3], 1, 1)));
        conv_current = conv_specs.back().get();
      }
      return conv_current;
    }
    default:
      break;
  }
  std::vector<int64_t> key;
  if (op.kind == OpKind::Conv2dNhwcFhwc || op.kind == OpKind::DepthwiseNhwcHwc) {
    const auto &ft = g.type(op.operands[1]).shape;
    const bool dw = op.kind == OpKind::DepthwiseNhwcHwc;
    key = {(int64_t)op.kind, ft[dw ? 0 : 1], ft[dw ? 1 : 2]};
  } else if (op.kind == OpKind::Transpose) {
    key = {(int64_t)op.kind};
    key.insert(key.end(), op.perm.begin(), op.perm.end());
  } else if (op.kind == OpKind::Generic && !op.results.empty()) {
    key = {(int64_t)op.kind, (int64_t)g.type(op.results[0]).shape.size()};
    key.insert(key.end(), op.iters.begin(), op.iters.end());
  } else {
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return &it->second;
  OperatorTilingSpec spec;
  if (op.kind == OpKind::Conv2dNhwcFhwc) spec = conv2d_nhwc_tiling_spec(key[1], key[2]);
  else if (op.kind == OpKind::DepthwiseNhwcHwc) spec = depthwise_nhwc_tiling_spec(key[1], key[2]);
  else if (op.kind == OpKind::Transpose)
    spec = transpose_tiling_spec(op.perm, (unsigned)op.perm.size());
  else
    spec = generic_tiling_spec(op.iters, (unsigned)key[1]);
  return &cache.emplace(key, std::move(spec)).first->second;
}

}  // namespace npu

namespace npu::ir {
const char *op_kind_name(OpKind k) {
  switch (k) {
    case OpKind::Matmul: return "linalg.matmul";
    case OpKind::BatchMatmul: return "linalg.batch_matmul";
    case OpKind::Conv2dNchwFchw: return "linalg.conv_2d_nchw_fchw";
    case OpKind::Conv2dNhwcFhwc: return "linalg.conv_2d_nhwc_fhwc";
    case OpKind::DepthwiseNhwcHwc: return "linalg.depthwise_conv_2d_nhwc_hwc";
    case OpKind::Generic: return "linalg.generic";
    case OpKind::Fill: return "linalg.fill";
    case OpKind::Transpose: return "linalg.transpose";
    case OpKind::Pad: return "tensor.pad";
    case OpKind::Empty: return "tensor.empty";
    case OpKind::Constant: return "arith.constant";
    case OpKind::Return: return "func.return";
    case OpKind::CollapseShape: return "tensor.collapse_shape";
    case OpKind::ExpandShape: return "tensor.expand_shape";
    case OpKind::Call: return "func.call";
    default: return "other";
  }
}
}  // namespace npu::ir
