// ir.hpp -- the MLIR-free program representation the cost model and the
// decision passes work on: a function body as SSA values and ops in block
// order, with the operand / result / user relations linalg exposes.
//
// For a linalg op, operands are its `ins` followed by its `outs` (DPS
// inits), as Operation::getOperands() returns them; `num_inputs` is the
// number of `ins`.  Non-linalg ops of the body (tensor.empty, tensor.pad,
// arith.constant, func.return, collapse/expand_shape) are ops too, so that
// "used outside a group" sees every user, e.g. the return.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace npu::ir {

enum class OpKind : int32_t {
  Matmul = 0,              // linalg.matmul
  BatchMatmul = 1,         // linalg.batch_matmul
  Conv2dNchwFchw = 2,      // linalg.conv_2d_nchw_fchw
  Conv2dNhwcFhwc = 3,      // linalg.conv_2d_nhwc_fhwc (authored here)
  DepthwiseNhwcHwc = 4,    // linalg.depthwise_conv_2d_nhwc_hwc (authored here)
  Generic = 5,             // linalg.generic
  Fill = 6,                // linalg.fill
  Transpose = 7,           // linalg.transpose
  Pad = 8,                 // tensor.pad
  Empty = 9,               // tensor.empty
  Constant = 10,           // arith.constant
  Return = 11,             // func.return
  CollapseShape = 12,      // tensor.collapse_shape
  ExpandShape = 13,        // tensor.expand_shape
  Call = 14,               // func.call
  Other = 15,
};

struct Type {
  std::vector<int64_t> shape;  // -1 = dynamic
  int32_t bits = 32;
  bool shaped = true;          // false for scalars (arith.constant operands of fill)
};

struct Value {
  Type type;
  int32_t def = -1;               // defining op (-1: function argument)
  std::vector<int32_t> users;     // one entry per use, in op order
};

struct Op {
  OpKind kind = OpKind::Other;
  std::vector<int32_t> operands;
  std::vector<int32_t> results;
  int32_t num_inputs = 0;         // linalg: number of `ins`
  std::vector<int32_t> iters;     // generic: 0 parallel, 1 reduction
  std::vector<int64_t> perm;      // transpose permutation
  std::vector<int64_t> strides;   // convolution strides (default 1)
};

struct Graph {
  std::vector<Value> values;
  std::vector<Op> ops;            // block order

  int32_t add_value(const Type &t) {
    values.push_back(Value{t, -1, {}});
    return (int32_t)values.size() - 1;
  }
  int32_t add_op(const Op &op) {
    const int32_t id = (int32_t)ops.size();
    ops.push_back(op);
    for (int32_t v : op.operands) values[v].users.push_back(id);
    for (int32_t v : op.results) values[v].def = id;
    return id;
  }
  const Type &type(int32_t v) const { return values[v].type; }
  bool is_linalg(int32_t op) const {
    switch (ops[op].kind) {
      case OpKind::Matmul: case OpKind::BatchMatmul: case OpKind::Conv2dNchwFchw:
      case OpKind::Conv2dNhwcFhwc: case OpKind::DepthwiseNhwcHwc: case OpKind::Generic:
      case OpKind::Fill: case OpKind::Transpose:
        return true;
      default:
        return false;
    }
  }
  // Operation::hasOneUse(): exactly one use of all results together.
  bool has_one_use(int32_t op) const {
    size_t uses = 0;
    for (int32_t r : ops[op].results) uses += values[r].users.size();
    return uses == 1;
  }
};

const char *op_kind_name(OpKind k);

}  // namespace npu::ir
