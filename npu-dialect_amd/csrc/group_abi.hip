// group_abi.hip -- npu_group_launch: the outlined-group boundary.
//
// A host module calls a fused group by the outliner's name with the group's
// external inputs in first-use order, then its results
// (lib/Transforms/OutlineFusedGroupsPass.cpp:218-263, 306-316).  This file
// reads those arguments -- MLIR memref descriptors of any rank plus the fill
// constant -- checks them against the group's signature, and runs the group
// through the typed entry points of abi.hip, which validate shapes again and
// launch.  No kernel lives here.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/npu_amd.h"
#include "plans.hpp"

namespace {

// The message of the first rejection; npu_group_launch hands it to
// npu_last_error() (a typed entry point's own message is copied here first).
thread_local std::string g_group_error;

npu_status gfail(npu_status code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_group_error = buf;
  return code;
}

// One argument read from its StridedMemRefType layout.
struct Arg {
  bool scalar = false;
  double value = 0.0;
  npu_memref m{};
};

npu_status read_arg(const npu_arg *a, int idx, const char *side, Arg *out) {
  if (a->kind == NPU_ARG_SCALAR) {
    out->scalar = true;
    out->value = a->scalar;
    return NPU_OK;
  }
  if (a->kind != NPU_ARG_MEMREF)
    return gfail(NPU_ERR_INVALID_ARG, "%s[%d]: kind %d is neither memref nor scalar", side, idx,
                 a->kind);
  if (a->rank < 1 || a->rank > NPU_MAX_RANK)
    return gfail(NPU_ERR_UNSUPPORTED, "%s[%d]: rank %lld (ranks 1..%d are taken)", side, idx,
                 (long long)a->rank, NPU_MAX_RANK);
  if (!a->descriptor) return gfail(NPU_ERR_INVALID_ARG, "%s[%d]: null descriptor", side, idx);
  // StridedMemRefType<T, R>: two pointers, then offset, sizes[R], strides[R].
  const char *d = static_cast<const char *>(a->descriptor);
  const int R = (int)a->rank;
  std::memcpy(&out->m.allocated, d, sizeof(void *));
  std::memcpy(&out->m.aligned, d + sizeof(void *), sizeof(void *));
  const int64_t *w = reinterpret_cast<const int64_t *>(d + 2 * sizeof(void *));
  out->m.offset = w[0];
  for (int i = 0; i < R; ++i) {
    out->m.sizes[i] = w[1 + i];
    out->m.strides[i] = w[1 + R + i];
  }
  out->m.rank = R;
  out->m.dtype = a->dtype;
  return NPU_OK;
}

bool same_shape(const npu_memref &m, std::initializer_list<int64_t> shape) {
  if (m.rank != (int)shape.size()) return false;
  int i = 0;
  for (int64_t s : shape)
    if (m.sizes[i++] != s) return false;
  return true;
}

std::string shape_str(const npu_memref &m) {
  std::string s = "[";
  for (int i = 0; i < m.rank; ++i) s += (i ? "," : "") + std::to_string((long long)m.sizes[i]);
  return s + "]";
}

// A view of a row-major [A,1,1,B] filter as [A,B].
npu_status squeeze_1x1(const npu_memref &m, const char *what, npu_memref *v) {
  if (m.strides[3] != 1 || (m.sizes[0] > 1 && m.strides[0] != m.sizes[3]))
    return gfail(NPU_ERR_UNSUPPORTED, "%s: only a row-major filter is supported", what);
  *v = m;
  v->rank = 2;
  v->sizes[0] = m.sizes[0];
  v->sizes[1] = m.sizes[3];
  v->strides[0] = m.sizes[3];
  v->strides[1] = 1;
  return NPU_OK;
}

// Chain key: each '+'-separated name without `fused_` and its `_<idx>`,
// joined by '_'.
std::string chain_key(const char *name) {
  std::string all(name), key;
  size_t start = 0;
  while (start <= all.size()) {
    size_t end = all.find('+', start);
    if (end == std::string::npos) end = all.size();
    std::string part = all.substr(start, end - start);
    if (part.rfind("fused_", 0) == 0) part = part.substr(6);
    const size_t us = part.rfind('_');
    if (us != std::string::npos && us + 1 < part.size() &&
        part.find_first_not_of("0123456789", us + 1) == std::string::npos)
      part = part.substr(0, us);
    if (!key.empty()) key += "_";
    key += part;
    start = end + 1;
  }
  return key;
}

class Cursor {
 public:
  Cursor(std::vector<Arg> &args) : a_(args) {}
  size_t pos() const { return i_; }
  size_t left() const { return a_.size() - i_; }
  bool done() const { return i_ == a_.size(); }
  const Arg *peek() const { return i_ < a_.size() ? &a_[i_] : nullptr; }
  // The fill constant: a scalar 0.0.
  npu_status fill_value() {
    if (done()) return gfail(NPU_ERR_INVALID_ARG, "in[%zu]: missing the fill value", i_);
    const Arg &x = a_[i_];
    if (!x.scalar)
      return gfail(NPU_ERR_INVALID_ARG, "in[%zu]: the fill value must be a scalar argument", i_);
    if (x.value != 0.0)
      return gfail(NPU_ERR_UNSUPPORTED, "in[%zu]: fill value %g (accumulators start at 0.0)", i_,
                   x.value);
    ++i_;
    return NPU_OK;
  }
  // A memref argument of the given rank.
  npu_status memref(int rank, const char *what, const npu_memref **m) {
    if (done()) return gfail(NPU_ERR_INVALID_ARG, "in[%zu]: missing %s", i_, what);
    const Arg &x = a_[i_];
    if (x.scalar || x.m.rank != rank)
      return gfail(NPU_ERR_INVALID_ARG, "in[%zu] (%s): expected a rank-%d memref", i_, what, rank);
    *m = &x.m;
    ++i_;
    return NPU_OK;
  }
  // A tensor.empty destination of exactly `shape`.
  npu_status dest(std::initializer_list<int64_t> shape, const char *what,
                  const npu_memref **m = nullptr) {
    const npu_memref *d;
    npu_status s = memref((int)shape.size(), what, &d);
    if (s != NPU_OK) return s;
    if (!same_shape(*d, shape))
      return gfail(NPU_ERR_INVALID_ARG, "in[%zu] (%s): shape %s does not match the group",
                   i_ - 1, what, shape_str(*d).c_str());
    if (m) *m = d;
    return NPU_OK;
  }
  // Optional rank-1 operand (a bias) when the next argument has rank 1.
  bool next_is_rank1() const { return peek() && !peek()->scalar && peek()->m.rank == 1; }

 private:
  std::vector<Arg> &a_;
  size_t i_ = 0;
};

#define G_TRY(expr)              \
  do {                           \
    npu_status _s = (expr);      \
    if (_s != NPU_OK) return _s; \
  } while (0)

// Keeps the launch plans of every typed call of a sequence (each call
// replaces the thread's plan list).
struct PlanLog {
  std::vector<npu_launch_plan> plans;
  void take() {
    const int n = npu_last_launch_plans(nullptr, 0);
    const size_t at = plans.size();
    plans.resize(at + n);
    npu_last_launch_plans(plans.data() + at, n);
  }
  void publish() {
    npu::plans_reset();
    for (const auto &p : plans) npu::plans_add(p);
  }
};

npu_status typed(npu_status s) {
  if (s != NPU_OK) g_group_error = npu_last_error();
  return s;
}

// chains[k]: whether matmul chain k ends in a generic (else its result is
// the accumulator the fill initialised, as the reference's last layers
// without an activation are).
npu_status run_matmuls(Cursor &c, const npu_group_attrs &at, const std::vector<bool> &gen,
                       const npu_memref *out, npu_stream stream, PlanLog &log) {
  const int chains = (int)gen.size();
  G_TRY(c.fill_value());
  const npu_memref *x = nullptr;
  struct Step { const npu_memref *init, *A, *B, *bias, *dest; };
  std::vector<Step> steps;
  for (int k = 0; k < chains; ++k) {
    Step s{};
    G_TRY(c.memref(2, "matmul accumulator (tensor.empty)", &s.init));
    if (k == 0) G_TRY(c.memref(2, "A", &x));
    s.A = x;
    G_TRY(c.memref(2, "B", &s.B));
    if (gen[k] && c.next_is_rank1()) G_TRY(c.memref(1, "bias", &s.bias));
    const int64_t M = s.A->sizes[0], N = s.B->sizes[1];
    // What each chain's typed call checks is checked here for every chain
    // first, so that no chain launches before all of them are known good.
    if (k == 0) G_TRY(typed(npu::memref_check(s.A, "A", 2, NPU_F32)));
    G_TRY(typed(npu::memref_check(s.B, "B", 2, NPU_F32)));
    if (s.bias) G_TRY(typed(npu::memref_check(s.bias, "bias", 1, NPU_F32)));
    if (s.B->sizes[0] != s.A->sizes[1])
      return gfail(NPU_ERR_INVALID_ARG, "matmul %d: B %s against A %s (K differs)", k,
                   shape_str(*s.B).c_str(), shape_str(*s.A).c_str());
    if (s.bias && s.bias->sizes[0] != N)
      return gfail(NPU_ERR_INVALID_ARG, "matmul %d: bias %s, expected [%lld]", k,
                   shape_str(*s.bias).c_str(), (long long)N);
    if (s.A->sizes[1] % 4 != 0)
      return gfail(NPU_ERR_UNSUPPORTED, "matmul %d: K = %lld (a multiple of 4 is required)", k,
                   (long long)s.A->sizes[1]);
    if (!same_shape(*s.init, {M, N}))
      return gfail(NPU_ERR_INVALID_ARG, "matmul %d: accumulator %s, expected [%lld,%lld]", k,
                   shape_str(*s.init).c_str(), (long long)M, (long long)N);
    if (gen[k])
      G_TRY(c.dest({M, N}, "generic destination (tensor.empty)", &s.dest));
    else
      s.dest = s.init;  // no generic: the result stays in the filled accumulator
    if (k + 1 < chains && !s.dest->aligned)
      return gfail(NPU_ERR_INVALID_ARG, "matmul %d: its destination holds the intermediate "
                   "result and must have data", k);
    if (k + 1 < chains) G_TRY(typed(npu::memref_check(s.dest, "intermediate destination", 2, NPU_F32)));
    steps.push_back(s);
    x = s.dest;  // the next chain reads this chain's result
  }
  if (!c.done())
    return gfail(NPU_ERR_INVALID_ARG, "%zu arguments left over after the group's inputs", c.pos());
  G_TRY(typed(npu::memref_check(out, "out", 2, NPU_F32)));
  if (!same_shape(*out, {steps.back().A->sizes[0], steps.back().B->sizes[1]}))
    return gfail(NPU_ERR_INVALID_ARG, "result %s: expected [%lld,%lld]", shape_str(*out).c_str(),
                 (long long)steps.back().A->sizes[0], (long long)steps.back().B->sizes[1]);
  for (int k = 0; k < chains; ++k) {
    const Step &s = steps[k];
    const npu_memref *dst = k + 1 == chains ? out : s.dest;
    npu_memref none{};
    none.rank = 1;
    G_TRY(typed(fused_matmul_bias_act(s.A, s.B, s.bias ? s.bias : &none, dst,
                                      gen[k] ? at.act[k] : NPU_ACT_NONE, stream)));
    log.take();
  }
  return NPU_OK;
}

// A conv group: fill, conv, then n_generic generics holding the epilogue
// (bias, residual, activation; an add and a ReLU may be two generics).  After
// (cst, init, x, w) come each generic's other operands and its destination,
// in first-use order.  A bias has rank 1; the residual and the destinations
// have the output's shape, the last destination last.  With one generic the
// residual is the rank-4 argument before the destination; with several,
// attrs.res_arg names its index in `in` (a bufferized host module passes
// allocated buffers for every destination), or, when it is 0, the
// destinations before the last must be passed without data (NULL) and the
// one rank-4 argument with data among them is the residual.
npu_status run_conv(Cursor &c, const npu_group_attrs &at, const npu_memref *out,
                    npu_stream stream, PlanLog &log, int n_generic, bool nchw) {
  G_TRY(c.fill_value());
  const npu_memref *init, *x, *w, *bias = nullptr;
  G_TRY(c.memref(4, "conv accumulator (tensor.empty)", &init));
  G_TRY(c.memref(4, "x", &x));
  G_TRY(c.memref(4, "w", &w));
  std::vector<const npu_memref *> r4;
  std::vector<size_t> r4_pos;
  while (!c.done()) {
    if (c.next_is_rank1()) {
      if (bias) return gfail(NPU_ERR_INVALID_ARG, "in[%zu]: a second bias", c.pos());
      G_TRY(c.memref(1, "bias", &bias));
    } else {
      const npu_memref *m;
      r4_pos.push_back(c.pos());
      G_TRY(c.memref(4, "residual or generic destination", &m));
      r4.push_back(m);
    }
  }
  const size_t nd = (size_t)n_generic;
  if (nd == 0 && (bias || !r4.empty()))
    return gfail(NPU_ERR_INVALID_ARG, "a conv group without a generic takes no bias, residual or "
                 "destination (its result is the filled accumulator)");
  if (r4.size() != nd && r4.size() != nd + 1)
    return gfail(NPU_ERR_INVALID_ARG, "%zu rank-4 arguments after the filter: expected %zu "
                 "destinations and at most one residual", r4.size(), nd);
  const npu_memref *res = nullptr;
  if (at.res_arg != 0) {
    for (size_t i = 0; i + 1 < r4.size(); ++i)
      if (r4_pos[i] == (size_t)at.res_arg) res = r4[i];
    if (!res || r4.size() != nd + 1)
      return gfail(NPU_ERR_INVALID_ARG, "res_arg %d does not name a rank-4 operand before the "
                   "last destination (with %zu generics)", at.res_arg, nd);
    if (!res->aligned) return gfail(NPU_ERR_INVALID_ARG, "the residual argument has no data");
  } else if (r4.size() == nd + 1) {
    if (nd == 1) {
      res = r4[0];
    } else {
      for (size_t i = 0; i + 1 < r4.size(); ++i)
        if (r4[i]->aligned) {
          if (res)
            return gfail(NPU_ERR_INVALID_ARG, "cannot tell the residual from the generics' "
                         "destinations: pass the destinations before the last without data");
          res = r4[i];
        }
      if (!res)
        return gfail(NPU_ERR_INVALID_ARG, "the residual argument has no data");
    }
  }
  for (const npu_memref *d : r4)
    if (d != res && !same_shape(*d, {out->sizes[0], out->sizes[1], out->sizes[2], out->sizes[3]}))
      return gfail(NPU_ERR_INVALID_ARG, "generic destination %s does not match the result %s",
                   shape_str(*d).c_str(), shape_str(*out).c_str());
  if (!same_shape(*init, {out->sizes[0], out->sizes[1], out->sizes[2], out->sizes[3]}))
    return gfail(NPU_ERR_INVALID_ARG, "conv accumulator %s does not match the result %s",
                 shape_str(*init).c_str(), shape_str(*out).c_str());
  npu_memref none{};
  none.rank = 1;
  if (nchw) {
    const int32_t st = at.stride > 1 ? at.stride : 1;
    if (res)
      G_TRY(typed(fused_conv2d_nchw_bias_res_act(x, w, bias ? bias : &none, res, out, at.pad, st,
                                                 at.act[0], stream)));
    else
      G_TRY(typed(fused_conv2d_nchw_bias_act(x, w, bias ? bias : &none, out, at.pad, st,
                                             at.act[0], stream)));
  } else if (at.stride > 1) {
    return gfail(NPU_ERR_UNSUPPORTED, "stride %d: the NHWC conv groups take stride 1", at.stride);
  } else if (res) {
    G_TRY(typed(fused_conv2d_nhwc_bias_res_act(x, w, bias ? bias : &none, res, out, at.pad,
                                               at.act[0], stream)));
  } else {
    G_TRY(typed(fused_conv2d_nhwc_bias_act(x, w, bias ? bias : &none, out, at.pad, at.act[0],
                                           stream)));
  }
  log.take();
  return NPU_OK;
}

npu_status run_irb(Cursor &c, const npu_memref *out, npu_stream stream, PlanLog &log) {
  G_TRY(c.fill_value());
  const npu_memref *init_e, *x, *we, *wdw, *wp;
  G_TRY(c.memref(4, "expand accumulator (tensor.empty)", &init_e));
  G_TRY(c.memref(4, "x", &x));
  G_TRY(c.memref(4, "we [E,1,1,C]", &we));
  const int64_t N = x->sizes[0], H = x->sizes[1], W = x->sizes[2], C = x->sizes[3];
  const int64_t E = we->sizes[0];
  if (!same_shape(*we, {E, 1, 1, C}))
    return gfail(NPU_ERR_INVALID_ARG, "we: %s, expected [E,1,1,%lld]", shape_str(*we).c_str(),
                 (long long)C);
  if (!same_shape(*init_e, {N, H, W, E}))
    return gfail(NPU_ERR_INVALID_ARG, "expand accumulator: %s", shape_str(*init_e).c_str());
  G_TRY(c.dest({N, H, W, E}, "expand destination (tensor.empty)"));
  G_TRY(c.dest({N, H, W, E}, "depthwise accumulator (tensor.empty)"));
  G_TRY(c.memref(3, "wdw [3,3,E]", &wdw));
  G_TRY(c.dest({N, H, W, E}, "depthwise destination (tensor.empty)"));
  G_TRY(c.dest({N, H, W, C}, "project accumulator (tensor.empty)"));
  G_TRY(c.memref(4, "wp [C,1,1,E]", &wp));
  if (!same_shape(*wp, {C, 1, 1, E}))
    return gfail(NPU_ERR_INVALID_ARG, "wp: %s, expected [%lld,1,1,%lld]", shape_str(*wp).c_str(),
                 (long long)C, (long long)E);
  G_TRY(c.dest({N, H, W, C}, "result destination (tensor.empty)"));
  if (!c.done())
    return gfail(NPU_ERR_INVALID_ARG, "%zu arguments left over after the group's inputs", c.pos());
  npu_memref we2, wp2;
  G_TRY(squeeze_1x1(*we, "we", &we2));
  G_TRY(squeeze_1x1(*wp, "wp", &wp2));
  G_TRY(typed(fused_irb_f32(x, &we2, wdw, &wp2, out, stream)));
  log.take();
  return NPU_OK;
}

npu_status run_qbottleneck(Cursor &c, const npu_memref *out, npu_stream stream, PlanLog &log) {
  G_TRY(c.fill_value());
  const npu_memref *x, *w1, *w2, *w3, *m1, *s1, *m2, *s2, *m3, *s3;
  const npu_memref *init1, *init2, *init3;
  G_TRY(c.memref(4, "conv1 accumulator (tensor.empty)", &init1));
  G_TRY(c.memref(4, "x", &x));
  G_TRY(c.memref(4, "w1 [M1,1,1,C]", &w1));
  const int64_t N = x->sizes[0], H = x->sizes[1], W = x->sizes[2], C = x->sizes[3];
  const int64_t M1 = w1->sizes[0];
  if (!same_shape(*w1, {M1, 1, 1, C}))
    return gfail(NPU_ERR_INVALID_ARG, "w1: %s, expected [M1,1,1,%lld]", shape_str(*w1).c_str(),
                 (long long)C);
  if (!same_shape(*init1, {N, H, W, M1}))
    return gfail(NPU_ERR_INVALID_ARG, "conv1 accumulator: %s", shape_str(*init1).c_str());
  G_TRY(c.memref(1, "m1", &m1));
  G_TRY(c.memref(1, "s1", &s1));
  G_TRY(c.dest({N, H, W, M1}, "y1 destination (tensor.empty)"));
  G_TRY(c.memref(4, "conv2 accumulator (tensor.empty)", &init2));
  if (!same_shape(*init2, {N, H, W, M1}))
    return gfail(NPU_ERR_INVALID_ARG, "conv2 accumulator: %s", shape_str(*init2).c_str());
  G_TRY(c.memref(4, "w2 [M1,3,3,M1]", &w2));
  G_TRY(c.memref(1, "m2", &m2));
  G_TRY(c.memref(1, "s2", &s2));
  G_TRY(c.dest({N, H, W, M1}, "y2 destination (tensor.empty)"));
  G_TRY(c.memref(4, "conv3 accumulator (tensor.empty)", &init3));
  if (!same_shape(*init3, {N, H, W, C}))
    return gfail(NPU_ERR_INVALID_ARG, "conv3 accumulator: %s", shape_str(*init3).c_str());
  G_TRY(c.memref(4, "w3 [C,1,1,M1]", &w3));
  if (!same_shape(*w3, {C, 1, 1, M1}))
    return gfail(NPU_ERR_INVALID_ARG, "w3: %s, expected [%lld,1,1,%lld]", shape_str(*w3).c_str(),
                 (long long)C, (long long)M1);
  G_TRY(c.memref(1, "m3", &m3));
  G_TRY(c.memref(1, "s3", &s3));
  G_TRY(c.dest({N, H, W, C}, "result destination (tensor.empty)"));
  if (!c.done())
    return gfail(NPU_ERR_INVALID_ARG, "%zu arguments left over after the group's inputs", c.pos());
  npu_memref w1v, w3v;
  G_TRY(squeeze_1x1(*w1, "w1", &w1v));
  G_TRY(squeeze_1x1(*w3, "w3", &w3v));
  G_TRY(typed(fused_qbottleneck_i8(x, &w1v, w2, &w3v, m1, s1, m2, s2, m3, s3, out, stream)));
  log.take();
  return NPU_OK;
}

const char *kConv = "fill_linalg_conv_2d_nhwc_fhwc";
// linalg.conv_2d_nchw_fchw's short name is `conv2d` (OutlineFusedGroupsPass.cpp:69-82)
const char *kConvNchw = "fill_conv2d";
const char *kQBottleneck =
    "fill_linalg_conv_2d_nhwc_fhwc_generic_fill_linalg_conv_2d_nhwc_fhwc_generic_"
    "fill_linalg_conv_2d_nhwc_fhwc_generic";
const char *kIrb =
    "fill_linalg_conv_2d_nhwc_fhwc_generic_fill_linalg_depthwise_conv_2d_nhwc_hwc_generic_"
    "fill_linalg_conv_2d_nhwc_fhwc_generic";

// The chains of a matmul group's key -- `fill_matmul` each, then `_generic`
// when the chain has an epilogue -- as one flag per chain; empty when the
// key is not such a sequence.
std::vector<bool> matmul_chains(const std::string &key) {
  const std::string one = "fill_matmul", gen = "_generic";
  std::vector<bool> chains;
  size_t p = 0;
  while (p < key.size()) {
    if (key.compare(p, one.size(), one) != 0) return {};
    p += one.size();
    bool g = false;
    if (key.compare(p, gen.size(), gen) == 0) {
      g = true;
      p += gen.size();
    }
    chains.push_back(g);
    if (p == key.size()) return chains;
    if (key[p] != '_') return {};
    ++p;
  }
  return {};
}

}  // namespace

extern "C" npu_status npu_group_launch(const char *outlined_name, const npu_group_attrs *attrs,
                                       const npu_arg *in, int32_t n_in, const npu_arg *out,
                                       int32_t n_out, npu_stream stream) {
  npu::plans_reset();
  g_group_error.clear();
  PlanLog log;
  npu_status st = [&]() -> npu_status {
    if (!outlined_name) return gfail(NPU_ERR_INVALID_ARG, "null group name");
    if (!attrs) return gfail(NPU_ERR_INVALID_ARG, "null group attributes");
    if (n_in < 0 || (n_in > 0 && !in)) return gfail(NPU_ERR_INVALID_ARG, "bad input list");
    if (n_out != 1 || !out)
      return gfail(NPU_ERR_UNSUPPORTED, "%d results (every group here returns one)", n_out);
    std::vector<Arg> args(n_in);
    for (int i = 0; i < n_in; ++i) G_TRY(read_arg(&in[i], i, "in", &args[i]));
    Arg res;
    G_TRY(read_arg(&out[0], 0, "out", &res));
    if (res.scalar) return gfail(NPU_ERR_INVALID_ARG, "out[0]: a result must be a memref");
    const std::string key = chain_key(outlined_name);
    Cursor c(args);
    const std::vector<bool> mm = matmul_chains(key);
    if (!mm.empty()) {
      if ((int)mm.size() > NPU_GROUP_MAX_CHAINS)
        return gfail(NPU_ERR_UNSUPPORTED, "%zu matmul chains (at most %d)", mm.size(),
                     NPU_GROUP_MAX_CHAINS);
      return run_matmuls(c, *attrs, mm, &res.m, stream, log);
    }
    // a conv followed by generics (none for the NCHW classifier convs), NHWC
    // (authored) or NCHW (the reference's own)
    for (const char *kc : {kConv, kConvNchw}) {
      if (key.rfind(kc, 0) != 0) continue;
      int ng = 0;
      size_t at = std::strlen(kc);
      while (key.compare(at, 8, "_generic") == 0 && key.size() >= at + 8) {
        ++ng;
        at += 8;
      }
      if (at == key.size() && (ng > 0 || kc == kConvNchw))
        return run_conv(c, *attrs, &res.m, stream, log, ng, kc == kConvNchw);
    }
    if (key == kIrb) return run_irb(c, &res.m, stream, log);
    if (key == kQBottleneck) return run_qbottleneck(c, &res.m, stream, log);
    return gfail(NPU_ERR_UNSUPPORTED, "no MI355X group runs the outlined chain '%s'", key.c_str());
  }();
  log.publish();
  if (st != NPU_OK) npu::set_last_error(g_group_error.c_str());
  return st;
}
