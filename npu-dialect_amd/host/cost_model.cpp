// cost_model.cpp -- analytical cost model over ir::Graph.
//
// The formulas restate lib/Analysis/CostModel.cpp (cited per function):
// decisions taken from them (fusion groups, tile sizes, spatial splits) have
// to agree with the reference's at its own target, so the arithmetic --
// integer divisions and casts included -- is kept alike.  Two differences,
// both outside the reference's op vocabulary: NHWC and depthwise
// convolutions get exact MAC counts and tile evaluations (the reference
// would count them as 1024 MACs), and sums that the reference could overflow
// (two "infinite" tile costs) saturate instead.
#include "cost_model.hpp"

#include <algorithm>
#include <cmath>
#include <limits>
#include <unordered_set>

namespace npu {

using ir::OpKind;

namespace {

constexpr int64_t kInf = std::numeric_limits<int64_t>::max() / 2;

int64_t sat_add(int64_t a, int64_t b) {
  if (a >= kInf || b >= kInf) return kInf;
  return std::min<int64_t>(a + b, kInf);
}

int64_t dim_or_one(const ir::Type &t, size_t d) {
  return (d < t.shape.size() && t.shape[d] >= 0) ? t.shape[d] : 1;
}

int64_t safe_product(const ir::Type &t) {
  int64_t p = 1;
  for (int64_t d : t.shape) p *= (d >= 0 ? d : 1);
  return p;
}

bool static_shape(const ir::Type &t) {
  if (!t.shaped) return false;
  for (int64_t d : t.shape)
    if (d < 0) return false;
  return true;
}

bool is_conv_like(OpKind k) {
  return k == OpKind::Conv2dNchwFchw || k == OpKind::Conv2dNhwcFhwc;
}

}  // namespace

bool ScheduleCost::valid() const { return total_cycles < kInf; }

int64_t HWTarget::inter_core_transfer_cycles(int64_t bytes) const {
  switch (interconnect) {
    case Interconnect::NoC:
      return noc_latency_cycles +
             std::max<int64_t>(1, static_cast<int64_t>(bytes / noc_bytes_per_cycle()));
    case Interconnect::SharedL1:
    case Interconnect::SharedSRAM:
      return 1;
    case Interconnect::DRAMOnly:
      return 2 * std::max<int64_t>(1, static_cast<int64_t>(bytes / bytes_per_cycle()));
  }
  return 0;
}

HWTarget mi355x_target(int32_t elem_bits) {
  HWTarget t;
  t.num_cores = 256;
  t.sram_per_core = 160 * 1024;
  t.clock_ghz = 2.4;
  t.dram_bandwidth = 31;                     // 8000 GB/s / 256 CUs
  t.sram_bandwidth = 307;                    // LDS 128 B/clk x 2.4 GHz
  t.matrix_throughput = elem_bits <= 8 ? 4096 : elem_bits <= 16 ? 2048 : 128;
  t.dsp_throughput = 64;                     // FP32 VALU lanes per CU
  t.dma_channels = 4;
  t.inter_core_sync_cost = 0;                // workgroups never wait on one another
  t.interconnect = Interconnect::SharedSRAM; // the L2 every CU of an XCD reads
  t.noc_bandwidth = 0;
  t.noc_latency_cycles = 0;
  t.shared_l1_size = 4 * 1024 * 1024;
  return t;
}

// ---------------------------------------------------------------- level 0
// CostModel.cpp:46-89
int64_t CostModel::op_macs(int32_t opi) const {
  const ir::Op &op = g_.ops[opi];
  // The output shape is the result's; an op in memref form has no result,
  // so its destination (the init operand, last) stands in for it.  The
  // reference reads getResult(0) for matmul / batch_matmul / conv, which such
  // an op does not have; a generic without results is priced at the default.
  const int32_t out = op.results.empty() ? (op.operands.empty() ? -1 : op.operands.back())
                                         : op.results[0];
  if (out < 0 && op.kind != OpKind::Generic) return 1024;
  switch (op.kind) {
    case OpKind::Matmul: {
      const auto &o = g_.type(out);
      const auto &a = g_.type(op.operands[0]);
      return dim_or_one(o, 0) * dim_or_one(o, 1) * dim_or_one(a, 1);
    }
    case OpKind::BatchMatmul: {
      const auto &o = g_.type(out);
      const auto &a = g_.type(op.operands[0]);
      return dim_or_one(o, 0) * dim_or_one(o, 1) * dim_or_one(o, 2) * dim_or_one(a, 2);
    }
    case OpKind::Conv2dNchwFchw: {
      const auto &o = g_.type(out);
      const auto &f = g_.type(op.operands[1]);
      return dim_or_one(o, 0) * dim_or_one(o, 1) * dim_or_one(o, 2) * dim_or_one(o, 3) *
             dim_or_one(f, 1) * dim_or_one(f, 2) * dim_or_one(f, 3);
    }
    case OpKind::Conv2dNhwcFhwc: {
      const auto &o = g_.type(out);
      const auto &f = g_.type(op.operands[1]);
      return safe_product(o) * dim_or_one(f, 1) * dim_or_one(f, 2) * dim_or_one(f, 3);
    }
    case OpKind::DepthwiseNhwcHwc: {
      const auto &o = g_.type(out);
      const auto &f = g_.type(op.operands[1]);
      return safe_product(o) * dim_or_one(f, 0) * dim_or_one(f, 1);
    }
    case OpKind::Generic:
      if (!op.results.empty()) return safe_product(g_.type(op.results[0]));
      break;
    default:
      break;
  }
  return 1024;
}

bool CostModel::is_matrix_op(int32_t opi) const {
  const OpKind k = g_.ops[opi].kind;
  return k == OpKind::Matmul || k == OpKind::BatchMatmul || is_conv_like(k);
}

// CostModel.cpp:91-101
int64_t CostModel::compute_cycles(int32_t op) const {
  const int64_t macs = op_macs(op);
  const int64_t tp = is_matrix_op(op) ? t_.matrix_throughput : t_.dsp_throughput;
  return std::max<int64_t>(1, macs / tp);
}

// CostModel.cpp:103-105
int64_t CostModel::dma_cycles(int64_t bytes) const {
  return std::max<int64_t>(1, static_cast<int64_t>(bytes / t_.bytes_per_cycle()));
}

// CostModel.cpp:107-113
int64_t CostModel::tensor_bytes(const ir::Type &t) {
  return safe_product(t) * std::max<int64_t>(1, t.bits / 8);
}

// ---------------------------------------------------------------- roofline
// CostModel.cpp:119-150.  The peak is the matrix (or DSP) rate times the
// clock: MAC/s of one core, compared with FLOPs.
RooflineCost CostModel::roofline_raw(double flops, double mem_bytes, bool matrix) const {
  RooflineCost c;
  c.flops = flops;
  c.mem_bytes = mem_bytes;
  const double peak = (matrix ? (double)t_.matrix_throughput : (double)t_.dsp_throughput) *
                      t_.clock_ghz * 1e9;
  const double bw = (double)t_.dram_bandwidth * 1e9;
  c.arithmetic_intensity = mem_bytes > 0 ? flops / mem_bytes : 1e12;
  const double ridge = peak / bw;
  c.peak_attainable = std::min(peak, c.arithmetic_intensity * bw);
  const double tc = peak > 0 ? flops / peak : 0;
  const double tm = bw > 0 ? mem_bytes / bw : 0;
  c.time_sec = std::max(tc, tm);
  c.memory_bound = c.arithmetic_intensity < ridge;
  c.efficiency = (peak > 0 && c.time_sec > 0) ? (flops / c.time_sec) / peak : 0;
  return c;
}

// CostModel.cpp:152-172: every operand and result goes to / from DRAM once.
RooflineCost CostModel::roofline(int32_t opi) const {
  const ir::Op &op = g_.ops[opi];
  const double flops = (double)op_macs(opi) * 2.0;
  double bytes = 0;
  for (int32_t v : op.operands)
    if (g_.type(v).shaped) bytes += (double)tensor_bytes(g_.type(v));
  for (int32_t v : op.results)
    if (g_.type(v).shaped) bytes += (double)tensor_bytes(g_.type(v));
  return roofline_raw(flops, bytes, is_matrix_op(opi));
}

// CostModel.cpp:174-226: only external operands (counted per use) and
// results used outside (or unused) cost DRAM bytes; intermediates stay on chip.
RooflineCost CostModel::roofline(const std::vector<int32_t> &ops) const {
  if (ops.empty()) return {};
  double flops = 0;
  for (int32_t op : ops) flops += (double)op_macs(op) * 2.0;
  std::unordered_set<int32_t> produced, in_set(ops.begin(), ops.end());
  for (int32_t op : ops)
    for (int32_t r : g_.ops[op].results) produced.insert(r);
  double bytes = 0;
  for (int32_t op : ops)
    for (int32_t v : g_.ops[op].operands)
      if (!produced.count(v) && g_.type(v).shaped) bytes += (double)tensor_bytes(g_.type(v));
  for (int32_t op : ops)
    for (int32_t r : g_.ops[op].results) {
      const auto &users = g_.values[r].users;
      bool outside = false;
      for (int32_t u : users)
        if (!in_set.count(u)) { outside = true; break; }
      if ((outside || users.empty()) && g_.type(r).shaped) bytes += (double)tensor_bytes(g_.type(r));
    }
  bool matrix = false;
  for (int32_t op : ops) {
    const OpKind k = g_.ops[op].kind;
    if (k == OpKind::Matmul || is_conv_like(k)) matrix = true;
  }
  return roofline_raw(flops, bytes, matrix);
}

// ---------------------------------------------------------------- level 1
// CostModel.cpp:232-274: double-buffered A and B, single C; pipelined tiles.
ScheduleCost CostModel::matmul_tile(int64_t tm, int64_t tn, int64_t tk, int64_t M, int64_t N,
                                    int64_t K, int64_t dtype_bytes, int64_t extra) const {
  const int64_t a = tm * tk * dtype_bytes, b = tk * tn * dtype_bytes, c = tm * tn * dtype_bytes;
  const int64_t peak = a * 2 + b * 2 + c + extra;
  if (peak > t_.sram_per_core) return {0, 0, kInf, peak, 0, 0};
  const int64_t tiles = ((M + tm - 1) / tm) * ((N + tn - 1) / tn) * ((K + tk - 1) / tk);
  const int64_t comp = std::max<int64_t>(1, (tm * tn * tk) / t_.matrix_throughput);
  const int64_t din = dma_cycles(a + b), dout = dma_cycles(c);
  const int64_t total = tiles <= 1 ? din + comp + dout
                                   : din + (tiles - 1) * std::max(din, comp) + comp + dout;
  return {tiles * comp, tiles * (din + dout), total, peak, tiles, tiles * (a + b + c)};
}

// CostModel.cpp:276-324: double-buffered input tile (with its Kh-1 / Kw-1
// halo), single filter and output tiles.
ScheduleCost CostModel::conv2d_tile(int64_t tn, int64_t tco, int64_t th, int64_t tw, int64_t N,
                                    int64_t Co, int64_t Ho, int64_t Wo, int64_t Ci, int64_t Kh,
                                    int64_t Kw, const std::vector<int64_t> &stride,
                                    int64_t dtype_bytes, int64_t extra_output_shaped) const {
  const int64_t sH = stride.size() > 0 ? stride[0] : 1, sW = stride.size() > 1 ? stride[1] : 1;
  const int64_t inH = std::min((th - 1) * sH + Kh, Ho * sH);
  const int64_t inW = std::min((tw - 1) * sW + Kw, Wo * sW);
  const int64_t in = tn * Ci * inH * inW * dtype_bytes;
  const int64_t w = tco * Ci * Kh * Kw * dtype_bytes;
  const int64_t out = tn * tco * th * tw * dtype_bytes;
  const int64_t peak = in * 2 + w + out + extra_output_shaped * out;
  if (peak > t_.sram_per_core) return {0, 0, kInf, peak, 0, 0};
  const int64_t tiles = ((N + tn - 1) / tn) * ((Co + tco - 1) / tco) * ((Ho + th - 1) / th) *
                        ((Wo + tw - 1) / tw);
  const int64_t comp =
      std::max<int64_t>(1, (tn * tco * th * tw * Ci * Kh * Kw) / t_.matrix_throughput);
  const int64_t din = dma_cycles(in + w), dout = dma_cycles(out);
  const int64_t total = tiles <= 1 ? din + comp + dout
                                   : din + (tiles - 1) * std::max(din, comp) + comp + dout;
  return {tiles * comp, tiles * (din + dout), total, peak, tiles, tiles * (in + w + out)};
}

// CostModel.cpp:330-340: halvings down to 16, then min(16, dim).
std::vector<int64_t> CostModel::tile_candidates(int64_t dim) {
  std::vector<int64_t> s;
  for (int64_t v = dim; v >= 16; v /= 2) s.push_back(v);
  if (s.empty() || s.back() > 16) s.push_back(std::min<int64_t>(16, dim));
  return s;
}

// ---------------------------------------------------------------- level 2
// CostModel.cpp:346-438
TileConfig CostModel::best_tile_config(int32_t opi) const {
  TileConfig best;
  best.cost = {0, 0, kInf, 0, 0, 0};
  const ir::Op &op = g_.ops[opi];
  if (op.results.empty()) return best;
  const ir::Type &out = g_.type(op.results[0]);
  const int64_t dtb = std::max<int64_t>(1, out.bits / 8);
  if (op.kind == OpKind::Matmul) {
    const int64_t M = out.shape[0], N = out.shape[1], K = g_.type(op.operands[0]).shape[1];
    for (int64_t tm : tile_candidates(M))
      for (int64_t tn : tile_candidates(N))
        for (int64_t tk : tile_candidates(K)) {
          const ScheduleCost c = matmul_tile(tm, tn, tk, M, N, K, dtb);
          if (c.total_cycles < best.cost.total_cycles) best = {{tm, tn, tk}, c};
        }
    return best;
  }
  if (is_conv_like(op.kind)) {
    const bool nhwc = op.kind == OpKind::Conv2dNhwcFhwc;
    const ir::Type &in = g_.type(op.operands[0]), &f = g_.type(op.operands[1]);
    const int64_t N_ = out.shape[0];
    const int64_t Co = nhwc ? out.shape[3] : out.shape[1];
    const int64_t Ho = nhwc ? out.shape[1] : out.shape[2];
    const int64_t Wo = nhwc ? out.shape[2] : out.shape[3];
    const int64_t Ci = nhwc ? in.shape[3] : in.shape[1];
    const int64_t Kh = nhwc ? f.shape[1] : f.shape[2], Kw = nhwc ? f.shape[2] : f.shape[3];
    const std::vector<int64_t> stride = {1, 1};
    const std::vector<int64_t> tns = N_ > 1 ? tile_candidates(N_) : std::vector<int64_t>{N_};
    for (int64_t tn : tns)
      for (int64_t tco : tile_candidates(Co))
        for (int64_t th : tile_candidates(Ho))
          for (int64_t tw : tile_candidates(Wo)) {
            const ScheduleCost c = conv2d_tile(tn, tco, th, tw, N_, Co, Ho, Wo, Ci, Kh, Kw, stride, dtb);
            if (c.total_cycles < best.cost.total_cycles) best = {{tn, tco, th, tw}, c};
          }
    return best;
  }
  if (op.kind == OpKind::Generic) {
    const int64_t dim0 = out.shape[0];
    int64_t per_row = 1;
    for (size_t i = 1; i < out.shape.size(); ++i) per_row *= out.shape[i];
    const int64_t bytes_per_row = per_row * dtb * 3;  // in + out + intermediate
    for (int64_t td : tile_candidates(dim0)) {
      const int64_t sram = td * bytes_per_row * 2;
      if (sram > t_.sram_per_core) continue;
      const int64_t tiles = (dim0 + td - 1) / td;
      const int64_t comp = std::max<int64_t>(1, (td * per_row) / t_.dsp_throughput);
      const int64_t dma = dma_cycles(td * bytes_per_row);
      const int64_t total = tiles <= 1 ? dma + comp + dma
                                       : dma + (tiles - 1) * std::max(dma, comp) + comp + dma;
      if (total < best.cost.total_cycles)
        best = {{td}, {tiles * comp, tiles * dma * 2, total, sram, tiles,
                       tiles * td * bytes_per_row * 2}};
    }
  }
  return best;
}

// CostModel.cpp:440-497
FusionDecision CostModel::fusion_profitable(int32_t producer, int32_t consumer) const {
  const OpKind ck = g_.ops[consumer].kind;
  if (ck == OpKind::Matmul || is_conv_like(ck)) return {false, 0};
  int32_t inter = -1;
  for (int32_t r : g_.ops[producer].results) {
    for (int32_t u : g_.values[r].users)
      if (u == consumer) { inter = r; break; }
    if (inter >= 0) break;
  }
  if (inter < 0 || !g_.type(inter).shaped) return {false, 0};
  const int64_t ib = tensor_bytes(g_.type(inter));
  const int64_t roundtrip = 2 * dma_cycles(ib);
  const ScheduleCost cp = best_tile_config(producer).cost, cc = best_tile_config(consumer).cost;
  const int64_t unfused = sat_add(sat_add(cp.total_cycles, cc.total_cycles), roundtrip);
  int64_t fused = sat_add(cp.total_cycles, cc.total_cycles);
  if (cp.sram_peak_bytes + ib > t_.sram_per_core) {
    const double ratio = (double)(cp.sram_peak_bytes + ib) / (double)t_.sram_per_core;
    fused = sat_add(fused, static_cast<int64_t>(roundtrip * (ratio - 1.0)));
  }
  const int64_t benefit = unfused - fused;
  return {benefit > 0, benefit};
}

// CostModel.cpp:499-566
ScheduleCost CostModel::spatial_split(int32_t opi, unsigned dim, int64_t chunks) const {
  const ir::Op &op = g_.ops[opi];
  if (op.results.empty()) return {0, 0, kInf, 0, 0, 0};
  const ir::Type &out = g_.type(op.results[0]);
  if (!static_shape(out) || dim >= out.shape.size()) return {0, 0, kInf, 0, 0, 0};
  const int64_t size = out.shape[dim];
  const int64_t active = std::min(chunks, size);
  if (active <= 0) return {0, 0, kInf, 0, 0, 0};
  const int64_t full = compute_cycles(opi);
  const int64_t comp = (full + active - 1) / active;
  int64_t in_bytes = 0;
  for (int32_t v : op.operands)
    if (g_.type(v).shaped) in_bytes += tensor_bytes(g_.type(v));
  int64_t per_core_bytes = in_bytes / active;
  if (op.operands.size() >= 2 && g_.type(op.operands[1]).shaped)
    per_core_bytes += tensor_bytes(g_.type(op.operands[1]));
  const int64_t dma = dma_cycles(per_core_bytes);
  const int64_t idle = active < chunks ? (chunks - active) * t_.inter_core_sync_cost : 0;
  int64_t total = std::max(comp, dma) + idle + t_.inter_core_sync_cost;
  const ScheduleCost tile = best_tile_config(opi).cost;
  const int64_t scaled = tile.valid() ? tile.total_cycles / std::max<int64_t>(1, active) : total;
  total = std::max(total, scaled);
  return {comp, dma, total, tile.sram_peak_bytes, tile.num_tiles, per_core_bytes * active};
}

// CostModel.cpp:568-677
TileAlignment CostModel::tile_alignment(const std::vector<int32_t> &ops) const {
  TileAlignment res{true, 0};
  if (ops.size() <= 1) return res;
  for (size_t i = 0; i + 1 < ops.size(); ++i) {
    const int32_t p = ops[i], c = ops[i + 1];
    int32_t conn = -1;
    for (int32_t r : g_.ops[p].results) {
      for (int32_t u : g_.values[r].users)
        if (u == c) { conn = r; break; }
      if (conn >= 0) break;
    }
    if (conn < 0) continue;
    if (!get_tiling_spec(g_, p) || !get_tiling_spec(g_, c)) continue;
    const ir::Type &ct = g_.type(conn);
    if (!static_shape(ct)) continue;
    if (g_.ops[c].results.empty()) continue;
    const ir::Type &co = g_.type(g_.ops[c].results[0]);
    if (!static_shape(co)) continue;
    if (ct.shape.size() != co.shape.size()) {
      res.aligned = false;
      res.overhead_bytes += tensor_bytes(ct);
      continue;
    }
    for (size_t d = 0; d < ct.shape.size(); ++d) {
      const int64_t pd = ct.shape[d], cd = co.shape[d];
      if (pd != cd && pd > 0 && cd > 0) {
        const int64_t eb = std::max<int64_t>(1, ct.bits / 8);
        int64_t elems = 1;
        for (int64_t x : ct.shape) elems *= x;
        const double ratio = (double)std::max(pd, cd) / (double)std::min(pd, cd);
        res.overhead_bytes += static_cast<int64_t>((ratio - 1.0) * elems * eb);
        res.aligned = false;
      }
    }
  }
  return res;
}

// CostModel.cpp:679-685
SpillStrategy CostModel::spill_strategy(int64_t ws, int64_t inter) const {
  const int64_t spill = 2 * dma_cycles(inter);
  const int64_t retile = dma_cycles(ws);
  return spill < retile ? SpillStrategy::Spill : SpillStrategy::Retile;
}

// CostModel.cpp:687-823
SpatialSplitCost CostModel::spatial_split_detailed(int32_t opi, const SplitDimSpec &spec,
                                                   int64_t chunks) const {
  SpatialSplitCost r;
  r.needs_reduce = !spec.parallel;
  const ir::Op &op = g_.ops[opi];
  if (op.results.empty()) return r;
  const ir::Type &out = g_.type(op.results[0]);
  if (!static_shape(out)) return r;
  int64_t size = 1;
  if (spec.output_dim < out.shape.size()) size = out.shape[spec.output_dim];
  const int64_t active = std::min(chunks, size);
  if (active <= 0) return r;
  const int64_t per_core_dim = (size + active - 1) / active;
  r.per_core_compute_cycles = (compute_cycles(opi) + active - 1) / active;
  for (const auto &rule : spec.input_rules) {
    if (rule.operand >= op.operands.size()) continue;
    const ir::Type &ot = g_.type(op.operands[rule.operand]);
    if (!ot.shaped) continue;
    const int64_t full = tensor_bytes(ot);
    switch (rule.kind) {
      case SliceKind::Shared:
        r.shared_data_bytes += full;
        r.per_core_dma_in_bytes += full;
        break;
      case SliceKind::Split: {
        int64_t sliced = full;
        if (rule.slice_dim < ot.shape.size()) {
          const int64_t orig = ot.shape[rule.slice_dim];
          if (orig > 0) sliced = full * per_core_dim / orig;
        }
        r.split_data_bytes += sliced;
        r.per_core_dma_in_bytes += sliced;
        break;
      }
      case SliceKind::Halo: {
        int64_t sliced = full;
        if (rule.slice_dim < ot.shape.size()) {
          const int64_t orig = ot.shape[rule.slice_dim];
          const int64_t halo = std::min(per_core_dim + rule.halo_low + rule.halo_high, orig);
          if (orig > 0) {
            sliced = full * halo / orig;
            r.halo_overhead_bytes += full * (rule.halo_low + rule.halo_high) / orig;
          }
        }
        r.split_data_bytes += sliced;
        r.per_core_dma_in_bytes += sliced;
        break;
      }
      case SliceKind::Reduce:
        r.per_core_dma_in_bytes += full;
        break;
    }
  }
  int64_t dma;
  if (r.shared_data_bytes > 0 && t_.interconnect != Interconnect::DRAMOnly) {
    const int64_t split_dma = dma_cycles(r.split_data_bytes + r.halo_overhead_bytes);
    const int64_t shared_load = dma_cycles(r.shared_data_bytes);
    const int64_t bcast = t_.inter_core_transfer_cycles(r.shared_data_bytes);
    dma = split_dma + std::max(shared_load / active, bcast);
  } else {
    dma = dma_cycles(r.per_core_dma_in_bytes);
  }
  int64_t reduce = 0;
  if (r.needs_reduce) {
    const int64_t ob = tensor_bytes(out);
    if (t_.interconnect == Interconnect::DRAMOnly) {
      reduce = (active - 1) * 2 * dma_cycles(ob);
    } else {
      int64_t steps = 1;
      for (int64_t c = active; c > 1; c /= 2) ++steps;
      reduce = steps * t_.inter_core_transfer_cycles(ob);
    }
  }
  const int64_t idle = active < chunks ? (chunks - active) * t_.inter_core_sync_cost : 0;
  r.total_cycles = std::max(r.per_core_compute_cycles, dma) + reduce + idle + t_.inter_core_sync_cost;
  return r;
}

// ---------------------------------------------------------------- level 3
// CostModel.cpp:829-932: three engines (DMA in, matrix, DSP) overlap in the
// steady state; DMA out drains.  Intermediates stay in SRAM.
SubgraphCost CostModel::subgraph(const std::vector<int32_t> &ops) const {
  SubgraphCost c;
  c.num_ops = (int64_t)ops.size();
  if (ops.empty()) return c;
  std::unordered_set<int32_t> produced, in_set(ops.begin(), ops.end());
  for (int32_t op : ops)
    for (int32_t r : g_.ops[op].results) produced.insert(r);
  for (int32_t op : ops) {
    const OpKind k = g_.ops[op].kind;
    const bool matrix = k == OpKind::Matmul || k == OpKind::BatchMatmul || is_conv_like(k);
    (matrix ? c.matrix_cycles : c.dsp_cycles) += compute_cycles(op);
  }
  std::vector<int32_t> ext_in;
  std::unordered_set<int32_t> seen_in;
  for (int32_t op : ops)
    for (int32_t v : g_.ops[op].operands)
      if (!produced.count(v) && seen_in.insert(v).second) ext_in.push_back(v);
  std::vector<int32_t> ext_out, inter;
  std::unordered_set<int32_t> out_set, inter_set;
  for (int32_t op : ops)
    for (int32_t r : g_.ops[op].results) {
      bool outside = false, inside = false;
      for (int32_t u : g_.values[r].users) (in_set.count(u) ? inside : outside) = true;
      if (outside || g_.values[r].users.empty()) {
        if (out_set.insert(r).second) ext_out.push_back(r);
      } else if (inside) {
        if (inter_set.insert(r).second) inter.push_back(r);
      }
    }
  for (int32_t r : g_.ops[ops.back()].results)
    if (!out_set.count(r)) {
      inter_set.erase(r);
      inter.erase(std::remove(inter.begin(), inter.end(), r), inter.end());
      out_set.insert(r);
      ext_out.push_back(r);
    }
  for (int32_t v : ext_in)
    if (g_.type(v).shaped) c.dma_in_cycles += dma_cycles(tensor_bytes(g_.type(v)));
  for (int32_t v : ext_out)
    if (g_.type(v).shaped) c.dma_out_cycles += dma_cycles(tensor_bytes(g_.type(v)));
  for (int32_t v : inter)
    if (g_.type(v).shaped) c.intermediate_dma += 2 * dma_cycles(tensor_bytes(g_.type(v)));
  c.unpipelined_cycles = c.dma_in_cycles + c.matrix_cycles + c.dsp_cycles + c.dma_out_cycles;
  c.pipelined_cycles = std::max({c.dma_in_cycles, c.matrix_cycles, c.dsp_cycles}) + c.dma_out_cycles;
  return c;
}

// CostModel.cpp:934-951
FusionDecision CostModel::subgraph_fusion_profitable(const std::vector<int32_t> &ops) const {
  if (ops.size() <= 1) return {false, 0};
  const int64_t fused = subgraph(ops).pipelined_cycles;
  int64_t unfused = 0;
  for (int32_t op : ops) unfused += subgraph({op}).pipelined_cycles;
  const int64_t benefit = unfused - fused;
  return {benefit > 0, benefit};
}

}  // namespace npu
