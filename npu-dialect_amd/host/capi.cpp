// capi.cpp -- extern "C" boundary of libnpu_host.so (include/npu_cost.h).
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/npu_cost.h"
#include "cost_model.hpp"
#include "memory_plan.hpp"
#include "passes.hpp"

namespace npu {
void gpu_params_mi355x(npu_gpu_params *p);
bool predict_launch(const npu_launch_plan &pl, const npu_gpu_params &g, npu_launch_cost *out);
}  // namespace npu

struct npu_graph {
  npu::ir::Graph g;
};

namespace {

thread_local std::string g_err;

int32_t fail(const char *fmt, ...) {
  char buf[256];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return -1;
}

npu::HWTarget to_target(const npu_hw_target *t) {
  npu::HWTarget h;
  h.num_cores = t->num_cores;
  h.sram_per_core = t->sram_per_core;
  h.dram_bandwidth = t->dram_bandwidth;
  h.sram_bandwidth = t->sram_bandwidth;
  h.matrix_throughput = t->matrix_throughput;
  h.dsp_throughput = t->dsp_throughput;
  h.dma_channels = t->dma_channels;
  h.inter_core_sync_cost = t->inter_core_sync_cost;
  h.clock_ghz = t->clock_ghz;
  h.interconnect = static_cast<npu::Interconnect>(t->interconnect);
  h.noc_bandwidth = t->noc_bandwidth;
  h.noc_latency_cycles = t->noc_latency_cycles;
  h.shared_l1_size = t->shared_l1_size;
  return h;
}

void from_target(const npu::HWTarget &h, npu_hw_target *t) {
  t->num_cores = h.num_cores;
  t->sram_per_core = h.sram_per_core;
  t->dram_bandwidth = h.dram_bandwidth;
  t->sram_bandwidth = h.sram_bandwidth;
  t->matrix_throughput = h.matrix_throughput;
  t->dsp_throughput = h.dsp_throughput;
  t->dma_channels = h.dma_channels;
  t->inter_core_sync_cost = h.inter_core_sync_cost;
  t->clock_ghz = h.clock_ghz;
  t->interconnect = static_cast<int32_t>(h.interconnect);
  t->reserved = 0;
  t->noc_bandwidth = h.noc_bandwidth;
  t->noc_latency_cycles = h.noc_latency_cycles;
  t->shared_l1_size = h.shared_l1_size;
}

bool bad_op(const npu_graph *g, int32_t op) {
  return !g || op < 0 || op >= (int32_t)g->g.ops.size();
}

bool bad_ops(const npu_graph *g, const int32_t *ops, int32_t n) {
  if (!g || (n > 0 && !ops) || n < 0) return true;
  for (int32_t i = 0; i < n; ++i)
    if (bad_op(g, ops[i])) return true;
  return false;
}

void put_schedule(const npu::ScheduleCost &c, const std::vector<int64_t> &tiles,
                  npu_schedule_cost *o) {
  o->compute_cycles = c.compute_cycles;
  o->dma_cycles = c.dma_cycles;
  o->total_cycles = c.total_cycles;
  o->sram_peak_bytes = c.sram_peak_bytes;
  o->num_tiles = c.num_tiles;
  o->total_dma_bytes = c.total_dma_bytes;
  o->valid = c.valid() ? 1 : 0;
  o->n_tile_sizes = (int32_t)std::min<size_t>(4, tiles.size());
  for (int i = 0; i < 4; ++i) o->tile_sizes[i] = i < (int)tiles.size() ? tiles[i] : 0;
}

void put_roofline(const npu::RooflineCost &c, npu_roofline *o) {
  o->flops = c.flops;
  o->mem_bytes = c.mem_bytes;
  o->arithmetic_intensity = c.arithmetic_intensity;
  o->time_sec = c.time_sec;
  o->is_memory_bound = c.memory_bound ? 1 : 0;
  o->reserved = 0;
  o->peak_attainable = c.peak_attainable;
  o->efficiency = c.efficiency;
}

std::vector<int32_t> vec(const int32_t *p, int32_t n) { return std::vector<int32_t>(p, p + n); }

}  // namespace

extern "C" {

void npu_hw_target_default(npu_hw_target *t) {
  if (t) from_target(npu::HWTarget{}, t);
}
void npu_hw_target_mi355x(npu_hw_target *t, int32_t bits) {
  if (t) from_target(npu::mi355x_target(bits), t);
}

npu_graph *npu_graph_create(void) { return new npu_graph(); }
void npu_graph_destroy(npu_graph *g) { delete g; }

int32_t npu_graph_add_value(npu_graph *g, const int64_t *shape, int32_t rank, int32_t bits,
                            int32_t shaped) {
  if (!g || rank < 0 || (rank > 0 && !shape) || bits <= 0) return fail("bad value");
  npu::ir::Type t;
  t.shape.assign(shape, shape + rank);
  t.bits = bits;
  t.shaped = shaped != 0;
  return g->g.add_value(t);
}

int32_t npu_graph_add_op(npu_graph *g, int32_t kind, const int32_t *operands, int32_t n_operands,
                         const int32_t *results, int32_t n_results, int32_t n_inputs,
                         const int32_t *iters, int32_t n_iters, const int64_t *perm,
                         int32_t n_perm) {
  if (!g || kind < 0 || kind > NPU_OP_OTHER) return fail("bad op kind %d", kind);
  const int32_t nv = (int32_t)g->g.values.size();
  for (int32_t i = 0; i < n_operands; ++i)
    if (operands[i] < 0 || operands[i] >= nv) return fail("operand %d: bad value id", i);
  for (int32_t i = 0; i < n_results; ++i)
    if (results[i] < 0 || results[i] >= nv || g->g.values[results[i]].def >= 0)
      return fail("result %d: bad or already defined value", i);
  npu::ir::Op op;
  op.kind = static_cast<npu::ir::OpKind>(kind);
  op.operands.assign(operands, operands + n_operands);
  op.results.assign(results, results + n_results);
  op.num_inputs = n_inputs;
  if (iters) op.iters.assign(iters, iters + n_iters);
  if (perm) op.perm.assign(perm, perm + n_perm);
  return g->g.add_op(op);
}

int32_t npu_graph_num_ops(const npu_graph *g) { return g ? (int32_t)g->g.ops.size() : -1; }

const char *npu_host_last_error(void) { return g_err.c_str(); }

namespace {
npu::SramBuffer from_c(const npu_sram_buffer &c) {
  npu::SramBuffer b;
  b.value = c.value;
  b.bytes = c.bytes;
  b.role = (npu::BufRole)c.role;
  b.first_use = c.first_use;
  b.last_use = c.last_use;
  b.in_loop = c.in_loop != 0;
  b.addr = c.addr;
  b.addr_pong = c.addr_pong;
  b.prefetch_addr = c.prefetch_addr;
  b.double_buffered = c.double_buffered != 0;
  b.spilled = c.spilled != 0;
  return b;
}
npu_sram_buffer to_c(const npu::SramBuffer &b) {
  npu_sram_buffer c;
  c.value = b.value;
  c.role = (int32_t)b.role;
  c.bytes = b.bytes;
  c.first_use = b.first_use;
  c.last_use = b.last_use;
  c.in_loop = b.in_loop;
  c.double_buffered = b.double_buffered;
  c.addr = b.addr;
  c.addr_pong = b.addr_pong;
  c.prefetch_addr = b.prefetch_addr;
  c.spilled = b.spilled;
  c.reserved = 0;
  return c;
}
}  // namespace

int32_t npu_pass_bufferize(const npu_graph *g, const int32_t *ops, int32_t n_ops,
                           const int64_t *bytes, int32_t n_bytes, npu_sram_buffer *out,
                           int32_t cap) {
  if (!g || (!ops && n_ops > 0) || n_ops < 0) return fail("bad arguments");
  std::vector<int32_t> v(ops, ops + n_ops);
  for (int32_t o : v)
    if (bad_op(g, o)) return fail("bad op %d", o);
  std::vector<int64_t> by;
  if (bytes && n_bytes > 0) by.assign(bytes, bytes + n_bytes);
  const auto bufs = npu::bufferize_loop(g->g, v, by.empty() ? nullptr : &by);
  for (size_t i = 0; i < bufs.size() && (int32_t)i < cap && out; ++i) out[i] = to_c(bufs[i]);
  return (int32_t)bufs.size();
}

int32_t npu_pass_sram_allocation(npu_sram_buffer *bufs, int32_t n, int64_t sram_size,
                                 npu_sram_summary *summary) {
  if ((!bufs && n > 0) || n < 0 || sram_size <= 0) return fail("bad arguments");
  std::vector<npu::SramBuffer> v;
  for (int32_t i = 0; i < n; ++i) {
    if (bufs[i].role < 0 || bufs[i].role > 2 || bufs[i].bytes < 0) return fail("bad buffer %d", i);
    npu::SramBuffer b = from_c(bufs[i]);
    b.addr = b.addr_pong = b.prefetch_addr = -1;
    b.double_buffered = b.spilled = false;
    v.push_back(b);
  }
  const npu::SramPlanSummary s = npu::plan_sram(v, sram_size);
  for (int32_t i = 0; i < n; ++i) bufs[i] = to_c(v[i]);
  if (summary) {
    summary->spilled = s.spilled;
    summary->prefetched = s.prefetched;
    summary->prefetch_bytes = s.prefetch_bytes;
    summary->peak_bytes = s.peak_bytes;
    summary->free_after = s.free_after;
  }
  return 0;
}

int32_t npu_pass_cost_evaluate(const npu_graph *g, const npu_hw_target *t, const int32_t *ops,
                               int32_t n_ops, const npu_sram_buffer *bufs, int32_t n_bufs,
                               int64_t tile_iterations, npu_kernel_cost *out) {
  if (!g || !t || !out || (!ops && n_ops > 0) || (!bufs && n_bufs > 0)) return fail("bad arguments");
  std::vector<int32_t> v(ops, ops + n_ops);
  for (int32_t o : v)
    if (bad_op(g, o)) return fail("bad op %d", o);
  std::vector<npu::SramBuffer> b;
  for (int32_t i = 0; i < n_bufs; ++i) b.push_back(from_c(bufs[i]));
  const npu::CostModel cm(g->g, to_target(t));
  const npu::KernelCost k = npu::cost_evaluate(g->g, cm, v, b, tile_iterations);
  out->flops = k.flops;
  out->mem_bytes = k.mem_bytes;
  out->arithmetic_intensity = k.arithmetic_intensity;
  out->time_sec = k.time_sec;
  out->efficiency = k.efficiency;
  out->memory_bound = k.memory_bound;
  out->reserved = 0;
  out->dma_in_bytes = k.dma_in_bytes;
  out->dma_out_bytes = k.dma_out_bytes;
  out->matrix_cycles = k.matrix_cycles;
  out->dsp_cycles = k.dsp_cycles;
  out->peak_sram_bytes = k.peak_sram_bytes;
  out->num_tile_iterations = k.num_tile_iterations;
  out->num_linalg_ops = k.num_linalg_ops;
  out->sram_budget = k.sram_budget;
  return 0;
}

void npu_gpu_params_mi355x(npu_gpu_params *p) {
  if (p) npu::gpu_params_mi355x(p);
}

int32_t npu_cm_predict_launch(const npu_launch_plan *plan, const npu_gpu_params *gpu,
                              npu_launch_cost *out) {
  if (!plan || !gpu || !out) return fail("null argument");
  if (!npu::predict_launch(*plan, *gpu, out))
    return fail("invalid launch plan '%.48s' (grid %d, tiles %d)", plan->kernel, plan->grid,
                plan->tiles);
  return 0;
}

int64_t npu_cm_op_macs(const npu_graph *g, const npu_hw_target *t, int32_t op) {
  if (bad_op(g, op) || !t) return fail("bad op");
  return npu::CostModel(g->g, to_target(t)).op_macs(op);
}
int64_t npu_cm_compute_cycles(const npu_graph *g, const npu_hw_target *t, int32_t op) {
  if (bad_op(g, op) || !t) return fail("bad op");
  return npu::CostModel(g->g, to_target(t)).compute_cycles(op);
}
int64_t npu_cm_dma_cycles(const npu_hw_target *t, int64_t bytes) {
  npu::ir::Graph empty;
  return npu::CostModel(empty, to_target(t)).dma_cycles(bytes);
}
int64_t npu_cm_tensor_bytes(const int64_t *shape, int32_t rank, int32_t bits) {
  npu::ir::Type ty;
  ty.shape.assign(shape, shape + rank);
  ty.bits = bits;
  return npu::CostModel::tensor_bytes(ty);
}

int32_t npu_cm_roofline_raw(const npu_hw_target *t, double flops, double bytes, int32_t matrix,
                            npu_roofline *out) {
  if (!t || !out) return fail("null argument");
  npu::ir::Graph empty;
  put_roofline(npu::CostModel(empty, to_target(t)).roofline_raw(flops, bytes, matrix != 0), out);
  return 0;
}

int32_t npu_cm_roofline(const npu_graph *g, const npu_hw_target *t, const int32_t *ops, int32_t n,
                        npu_roofline *out) {
  if (bad_ops(g, ops, n) || !t || !out) return fail("bad ops");
  npu::CostModel cm(g->g, to_target(t));
  put_roofline(n == 1 ? cm.roofline(ops[0]) : cm.roofline(vec(ops, n)), out);
  return 0;
}

int32_t npu_cm_matmul_tile(const npu_hw_target *t, int64_t tm, int64_t tn, int64_t tk, int64_t M,
                           int64_t N, int64_t K, int64_t dtb, int64_t extra,
                           npu_schedule_cost *out) {
  if (!t || !out || tm <= 0 || tn <= 0 || tk <= 0) return fail("bad tile");
  npu::ir::Graph empty;
  put_schedule(npu::CostModel(empty, to_target(t)).matmul_tile(tm, tn, tk, M, N, K, dtb, extra),
               {tm, tn, tk}, out);
  return 0;
}

int32_t npu_cm_conv2d_tile(const npu_hw_target *t, int64_t tn, int64_t tco, int64_t th, int64_t tw,
                           int64_t N, int64_t Co, int64_t Ho, int64_t Wo, int64_t Ci, int64_t Kh,
                           int64_t Kw, int64_t sh, int64_t sw, int64_t dtb, int64_t extra,
                           npu_schedule_cost *out) {
  if (!t || !out || tn <= 0 || tco <= 0 || th <= 0 || tw <= 0) return fail("bad tile");
  npu::ir::Graph empty;
  put_schedule(npu::CostModel(empty, to_target(t))
                   .conv2d_tile(tn, tco, th, tw, N, Co, Ho, Wo, Ci, Kh, Kw, {sh, sw}, dtb, extra),
               {tn, tco, th, tw}, out);
  return 0;
}

int32_t npu_spec_reset(void) {
  npu::reset_conv_spec();
  return 0;
}

int32_t npu_cm_tile_candidates(int64_t dim, int64_t *out, int32_t cap) {
  const auto c = npu::CostModel::tile_candidates(dim);
  for (int32_t i = 0; i < cap && i < (int32_t)c.size(); ++i) out[i] = c[i];
  return (int32_t)c.size();
}

int32_t npu_cm_best_tile_config(const npu_graph *g, const npu_hw_target *t, int32_t op,
                                npu_schedule_cost *out) {
  if (bad_op(g, op) || !t || !out) return fail("bad op");
  const npu::TileConfig c = npu::CostModel(g->g, to_target(t)).best_tile_config(op);
  put_schedule(c.cost, c.tile_sizes, out);
  return 0;
}

int32_t npu_cm_fusion_profitable(const npu_graph *g, const npu_hw_target *t, int32_t producer,
                                 int32_t consumer, int64_t *benefit) {
  if (bad_op(g, producer) || bad_op(g, consumer) || !t) return fail("bad op");
  const auto d = npu::CostModel(g->g, to_target(t)).fusion_profitable(producer, consumer);
  if (benefit) *benefit = d.benefit_cycles;
  return d.fuse ? 1 : 0;
}

int32_t npu_cm_spatial_split(const npu_graph *g, const npu_hw_target *t, int32_t op, int32_t dim,
                             int64_t chunks, npu_schedule_cost *out) {
  if (bad_op(g, op) || !t || !out || dim < 0) return fail("bad op");
  put_schedule(npu::CostModel(g->g, to_target(t)).spatial_split(op, (unsigned)dim, chunks), {}, out);
  return 0;
}

int32_t npu_cm_spatial_split_detailed(const npu_graph *g, const npu_hw_target *t, int32_t op,
                                      int32_t idx, int64_t chunks, npu_spatial_split_cost *out) {
  if (bad_op(g, op) || !t || !out) return fail("bad op");
  const npu::OperatorTilingSpec *spec = npu::get_tiling_spec(g->g, op);
  if (!spec || idx < 0 || idx >= (int32_t)spec->split_dims.size()) return fail("bad split index");
  const auto r = npu::CostModel(g->g, to_target(t)).spatial_split_detailed(op, spec->split_dims[idx], chunks);
  out->per_core_dma_in_bytes = r.per_core_dma_in_bytes;
  out->per_core_compute_cycles = r.per_core_compute_cycles;
  out->shared_data_bytes = r.shared_data_bytes;
  out->split_data_bytes = r.split_data_bytes;
  out->halo_overhead_bytes = r.halo_overhead_bytes;
  out->needs_reduce = r.needs_reduce ? 1 : 0;
  out->reserved = 0;
  out->total_cycles = r.total_cycles;
  return 0;
}

int32_t npu_cm_tile_alignment(const npu_graph *g, const npu_hw_target *t, const int32_t *ops,
                              int32_t n, int64_t *overhead) {
  if (bad_ops(g, ops, n) || !t) return fail("bad ops");
  const auto a = npu::CostModel(g->g, to_target(t)).tile_alignment(vec(ops, n));
  if (overhead) *overhead = a.overhead_bytes;
  return a.aligned ? 1 : 0;
}

int32_t npu_cm_spill_strategy(const npu_hw_target *t, int64_t ws, int64_t inter) {
  npu::ir::Graph empty;
  return (int32_t)npu::CostModel(empty, to_target(t)).spill_strategy(ws, inter);
}

int32_t npu_cm_subgraph(const npu_graph *g, const npu_hw_target *t, const int32_t *ops, int32_t n,
                        npu_subgraph_cost *out) {
  if (bad_ops(g, ops, n) || !t || !out) return fail("bad ops");
  const auto c = npu::CostModel(g->g, to_target(t)).subgraph(vec(ops, n));
  out->dma_in_cycles = c.dma_in_cycles;
  out->matrix_cycles = c.matrix_cycles;
  out->dsp_cycles = c.dsp_cycles;
  out->dma_out_cycles = c.dma_out_cycles;
  out->intermediate_dma = c.intermediate_dma;
  out->pipelined_cycles = c.pipelined_cycles;
  out->unpipelined_cycles = c.unpipelined_cycles;
  out->num_ops = c.num_ops;
  return 0;
}

int32_t npu_cm_subgraph_fusion_profitable(const npu_graph *g, const npu_hw_target *t,
                                          const int32_t *ops, int32_t n, int64_t *benefit) {
  if (bad_ops(g, ops, n) || !t) return fail("bad ops");
  const auto d = npu::CostModel(g->g, to_target(t)).subgraph_fusion_profitable(vec(ops, n));
  if (benefit) *benefit = d.benefit_cycles;
  return d.fuse ? 1 : 0;
}

int32_t npu_spec_num_splits(const npu_graph *g, int32_t op) {
  if (bad_op(g, op)) return fail("bad op");
  const npu::OperatorTilingSpec *s = npu::get_tiling_spec(g->g, op);
  return s ? (int32_t)s->split_dims.size() : 0;
}

int32_t npu_spec_split(const npu_graph *g, int32_t op, int32_t index, int32_t *output_dim,
                       int32_t *iter_dim, int32_t *parallel) {
  if (bad_op(g, op)) return fail("bad op");
  const npu::OperatorTilingSpec *s = npu::get_tiling_spec(g->g, op);
  if (!s || index < 0 || index >= (int32_t)s->split_dims.size()) return fail("bad split index");
  const auto &d = s->split_dims[index];
  if (output_dim) *output_dim = d.output_dim == npu::kNoOutputDim ? -1 : (int32_t)d.output_dim;
  if (iter_dim) *iter_dim = (int32_t)d.iter_dim;
  if (parallel) *parallel = d.parallel ? 1 : 0;
  return 0;
}

int32_t npu_spec_preferred_spatial_dim(const npu_graph *g, int32_t op) {
  if (bad_op(g, op)) return fail("bad op");
  const npu::OperatorTilingSpec *s = npu::get_tiling_spec(g->g, op);
  return s ? s->preferred_spatial_dim : -1;
}

static int32_t put_groups(const std::vector<std::vector<int32_t>> &groups, int32_t *ops_out,
                          int32_t cap_ops, int32_t *sizes_out, int32_t cap_groups) {
  int32_t k = 0;
  for (size_t i = 0; i < groups.size(); ++i) {
    if ((int32_t)i < cap_groups && sizes_out) sizes_out[i] = (int32_t)groups[i].size();
    for (int32_t op : groups[i]) {
      if (k < cap_ops && ops_out) ops_out[k] = op;
      ++k;
    }
  }
  return (int32_t)groups.size();
}

int32_t npu_pass_fusion_groups(const npu_graph *g, const npu_hw_target *t, int32_t *ops_out,
                               int32_t cap_ops, int32_t *sizes_out, int32_t cap_groups) {
  if (!g || !t) return fail("null argument");
  npu::CostModel cm(g->g, to_target(t));
  return put_groups(npu::fusion_groups(g->g, cm), ops_out, cap_ops, sizes_out, cap_groups);
}

int32_t npu_pass_tile_and_fuse(const npu_graph *g, const npu_hw_target *t, int32_t consumer,
                               npu_schedule_cost *out) {
  if (bad_op(g, consumer) || !t || !out) return fail("bad op");
  npu::CostModel cm(g->g, to_target(t));
  npu::TileConfig c;
  const bool tiled = npu::tile_and_fuse_decision(g->g, cm, consumer, &c);
  put_schedule(c.cost, c.tile_sizes, out);
  return tiled ? 1 : 0;
}

static std::vector<npu::OutlinedGroup> outline_all(const npu_graph *g, const npu::CostModel &cm) {
  std::vector<int32_t> scope(g->g.ops.size());
  for (size_t i = 0; i < scope.size(); ++i) scope[i] = (int32_t)i;
  return npu::outline_groups(g->g, cm, scope);
}

int32_t npu_pass_outline_groups(const npu_graph *g, const npu_hw_target *t, int32_t *ops_out,
                                int32_t cap_ops, int32_t *sizes_out, int32_t cap_groups) {
  if (!g || !t) return fail("null argument");
  npu::CostModel cm(g->g, to_target(t));
  std::vector<std::vector<int32_t>> groups;
  for (const auto &grp : outline_all(g, cm)) groups.push_back(grp.ops);
  return put_groups(groups, ops_out, cap_ops, sizes_out, cap_groups);
}

int32_t npu_pass_outline_group_info(const npu_graph *g, const npu_hw_target *t, int32_t index,
                                    char *name, int32_t name_cap, int32_t *inputs,
                                    int32_t *n_inputs, int32_t *outputs, int32_t *n_outputs,
                                    int32_t cap) {
  if (!g || !t) return fail("null argument");
  npu::CostModel cm(g->g, to_target(t));
  const auto groups = outline_all(g, cm);
  if (index < 0 || index >= (int32_t)groups.size()) return fail("bad group index %d", index);
  const auto &grp = groups[index];
  if (name && name_cap > 0) {
    const size_t n = std::min<size_t>(grp.name.size(), (size_t)name_cap - 1);
    std::copy(grp.name.begin(), grp.name.begin() + n, name);
    name[n] = '\0';
  }
  if (n_inputs) *n_inputs = (int32_t)grp.inputs.size();
  if (n_outputs) *n_outputs = (int32_t)grp.outputs.size();
  for (int32_t i = 0; i < cap && i < (int32_t)grp.inputs.size(); ++i)
    if (inputs) inputs[i] = grp.inputs[i];
  for (int32_t i = 0; i < cap && i < (int32_t)grp.outputs.size(); ++i)
    if (outputs) outputs[i] = grp.outputs[i];
  return 0;
}

int32_t npu_pass_spatial(const npu_graph *g, const npu_hw_target *t, int32_t op, int64_t cores,
                         npu_spatial_decision *out) {
  if (bad_op(g, op) || !t || !out || cores <= 0) return fail("bad argument");
  npu::CostModel cm(g->g, to_target(t));
  npu::SpatialDecision d;
  const bool tiled = npu::spatial_decision(g->g, cm, op, cores, &d);
  *out = npu_spatial_decision{};
  if (!tiled) return 0;
  out->iter_dim = d.iter_dim;
  out->out_dim = d.out_dim;
  out->dim_size = d.dim_size;
  out->tile_size = d.tile_size;
  out->full_iters = d.full_iters;
  out->peel_size = d.peel_size;
  out->cost = d.cost;
  out->n_candidates = (int32_t)std::min<size_t>(8, d.candidates.size());
  for (int32_t i = 0; i < out->n_candidates; ++i) {
    out->cand_iter_dims[i] = d.candidates[i].first;
    out->cand_costs[i] = d.candidates[i].second;
  }
  return 1;
}

int32_t npu_pass_temporal(const npu_graph *g, const npu_hw_target *t, int32_t op,
                          npu_schedule_cost *cost, int64_t *tile_sizes, int32_t cap) {
  if (bad_op(g, op) || !t) return fail("bad argument");
  npu::CostModel cm(g->g, to_target(t));
  npu::TileConfig c;
  if (!npu::temporal_decision(g->g, cm, op, &c)) return 0;
  if (cost) put_schedule(c.cost, c.tile_sizes, cost);
  for (int32_t i = 0; i < cap && i < (int32_t)c.tile_sizes.size(); ++i)
    if (tile_sizes) tile_sizes[i] = c.tile_sizes[i];
  return (int32_t)c.tile_sizes.size();
}

int32_t npu_pass_barrier_alloc(const int32_t *kinds, int32_t n, int64_t pool, int64_t *subgraph,
                               int64_t *barrier_id, int64_t *generation) {
  if (pool < 1 || n < 0 || (n > 0 && (!kinds || !subgraph || !barrier_id || !generation)))
    return fail("barrier alloc: pool must be >= 1 and the arrays non-null");
  std::vector<npu::SchedKind> ops(n);
  for (int32_t i = 0; i < n; ++i)
    ops[i] = kinds[i] >= 0 && kinds[i] <= 2 ? static_cast<npu::SchedKind>(kinds[i]) : npu::SchedKind::Ignore;
  const auto a = npu::barrier_alloc(ops, pool);
  int64_t subs = 0;
  for (int32_t i = 0; i < n; ++i) {
    subgraph[i] = a[i].subgraph;
    barrier_id[i] = a[i].barrier_id;
    generation[i] = a[i].generation;
    subs = std::max<int64_t>(subs, a[i].subgraph + 1);
  }
  return (int32_t)subs;
}

}  // extern "C"
