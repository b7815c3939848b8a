// passes.cpp -- decision logic of npu-fusion, npu-outline-fused-groups,
// npu-spatial-tiling and npu-temporal-tiling over ir::Graph.
#include "passes.hpp"

#include <algorithm>
#include <limits>
#include <numeric>
#include <unordered_map>
#include <unordered_set>

namespace npu {

using ir::OpKind;

namespace {

constexpr int64_t kInf = std::numeric_limits<int64_t>::max() / 2;

bool is_compute(const ir::Graph &g, int32_t op) {
  return g.is_linalg(op) && g.ops[op].kind != OpKind::Fill;
}

bool contains(const std::vector<int32_t> &v, int32_t x) {
  return std::find(v.begin(), v.end(), x) != v.end();
}

// FusionPass.cpp:65-86
std::vector<int32_t> single_use_consumers(const ir::Graph &g, int32_t op,
                                          const std::unordered_set<int32_t> &set) {
  std::vector<int32_t> out;
  for (int32_t r : g.ops[op].results) {
    const auto &users = g.values[r].users;
    if (users.size() != 1) continue;
    const int32_t u = users[0];
    if (is_reshape_boundary(g, u)) continue;
    if (set.count(u) && is_compute(g, u)) out.push_back(u);
  }
  return out;
}

// FusionPass.cpp:88-109
std::vector<int32_t> single_use_producers(const ir::Graph &g, int32_t op,
                                          const std::unordered_set<int32_t> &set) {
  std::vector<int32_t> out;
  for (int32_t v : g.ops[op].operands) {
    const int32_t d = g.values[v].def;
    if (d < 0 || is_reshape_boundary(g, d) || !set.count(d) || !is_compute(g, d)) continue;
    if (!g.has_one_use(d)) continue;
    out.push_back(d);
  }
  return out;
}

// FusionPass.cpp:113-126
bool shapes_compatible(const ir::Graph &g, int32_t producer, int32_t consumer) {
  for (int32_t r : g.ops[producer].results)
    for (int32_t u : g.values[r].users)
      if (u == consumer) {
        const ir::Type &t = g.type(r);
        if (!t.shaped) return false;
        for (int64_t d : t.shape)
          if (d < 0) return false;
        return true;
      }
  return false;
}

bool aligned_enough(const CostModel &cm, int32_t a, int32_t b) {
  const TileAlignment al = cm.tile_alignment({a, b});
  return al.aligned || al.overhead_bytes <= cm.target().sram_per_core / 4;
}

int64_t group_benefit(const CostModel &cm, const std::vector<int32_t> &group,
                      const std::vector<int32_t> &trial, int32_t cand) {
  const int64_t fused = cm.subgraph(trial).pipelined_cycles;
  const int64_t unfused = cm.subgraph(group).pipelined_cycles + cm.subgraph({cand}).pipelined_cycles;
  return unfused - fused;
}

// Iteration-domain extents per op kind (the loop order of the linalg op).
std::vector<int64_t> iter_sizes(const ir::Graph &g, int32_t opi) {
  const ir::Op &op = g.ops[opi];
  const auto &o = g.type(op.results[0]).shape;
  switch (op.kind) {
    case OpKind::Matmul:
      return {o[0], o[1], g.type(op.operands[0]).shape[1]};
    case OpKind::BatchMatmul:
      return {o[0], o[1], o[2], g.type(op.operands[0]).shape[2]};
    case OpKind::Conv2dNchwFchw: {
      const auto &f = g.type(op.operands[1]).shape;
      return {o[0], o[1], o[2], o[3], f[1], f[2], f[3]};
    }
    case OpKind::Conv2dNhwcFhwc: {
      const auto &f = g.type(op.operands[1]).shape;
      return {o[0], o[1], o[2], o[3], f[1], f[2], f[3]};
    }
    case OpKind::DepthwiseNhwcHwc: {
      const auto &f = g.type(op.operands[1]).shape;
      return {o[0], o[1], o[2], o[3], f[0], f[1]};
    }
    case OpKind::Generic: {
      std::vector<int64_t> s(op.iters.size(), 1);
      for (int32_t v : op.operands) {
        const ir::Type &t = g.type(v);
        if (!t.shaped || t.shape.size() != s.size()) continue;
        for (size_t d = 0; d < s.size(); ++d)
          if (t.shape[d] > 0) s[d] = std::max(s[d], t.shape[d]);
      }
      return s;
    }
    default:
      return std::vector<int64_t>(o.begin(), o.end());
  }
}

size_t num_loops(const ir::Graph &g, int32_t op) { return iter_sizes(g, op).size(); }

}  // namespace

std::vector<std::vector<int32_t>> fusion_groups(const ir::Graph &g, const CostModel &cm) {
  std::vector<int32_t> all;
  for (int32_t i = 0; i < (int32_t)g.ops.size(); ++i)
    if (is_compute(g, i)) all.push_back(i);
  std::unordered_set<int32_t> set(all.begin(), all.end());
  std::vector<std::pair<int64_t, int32_t>> order;
  for (int32_t op : all) order.push_back({cm.compute_cycles(op), op});
  std::stable_sort(order.begin(), order.end(),
                   [](const auto &a, const auto &b) { return a.first > b.first; });
  std::unordered_set<int32_t> visited;
  std::vector<std::vector<int32_t>> groups;
  for (const auto &[cost, anchor] : order) {
    (void)cost;
    if (visited.count(anchor)) continue;
    std::vector<int32_t> group = {anchor};
    while (group.size() < kMaxFusionLength) {  // forward: consumers of the last op
      const int32_t last = group.back();
      int32_t best = -1;
      int64_t best_benefit = 0;
      for (int32_t c : single_use_consumers(g, last, set)) {
        if (visited.count(c) || contains(group, c)) continue;
        if (!shapes_compatible(g, last, c) || !aligned_enough(cm, last, c)) continue;
        std::vector<int32_t> trial = group;
        trial.push_back(c);
        const int64_t b = group_benefit(cm, group, trial, c);
        if (b > best_benefit) { best = c; best_benefit = b; }
      }
      if (best < 0) break;
      group.push_back(best);
    }
    while (group.size() < kMaxFusionLength) {  // backward: producers of the first op
      const int32_t first = group.front();
      int32_t best = -1;
      int64_t best_benefit = 0;
      for (int32_t p : single_use_producers(g, first, set)) {
        if (visited.count(p) || contains(group, p)) continue;
        if (!shapes_compatible(g, p, first) || !aligned_enough(cm, p, first)) continue;
        std::vector<int32_t> trial = {p};
        trial.insert(trial.end(), group.begin(), group.end());
        const int64_t b = group_benefit(cm, group, trial, p);
        if (b > best_benefit) { best = p; best_benefit = b; }
      }
      if (best < 0) break;
      group.insert(group.begin(), best);
    }
    for (int32_t op : group) visited.insert(op);
    if (group.size() > 1) groups.push_back(group);
  }
  return groups;
}

bool tile_and_fuse_decision(const ir::Graph &g, const CostModel &cm, int32_t consumer,
                            TileConfig *config) {
  *config = cm.best_tile_config(consumer);
  (void)g;
  return !config->tile_sizes.empty() && config->cost.valid() && config->cost.num_tiles > 1;
}

std::string short_op_name(const ir::Graph &g, int32_t op) {
  switch (g.ops[op].kind) {
    case OpKind::Matmul: return "matmul";
    case OpKind::Conv2dNchwFchw: return "conv2d";
    case OpKind::Fill: return "fill";
    case OpKind::Generic: return "generic";
    default: {
      std::string n = ir::op_kind_name(g.ops[op].kind);
      std::replace(n.begin(), n.end(), '.', '_');
      return n;
    }
  }
}

std::vector<OutlinedGroup> outline_groups(const ir::Graph &g, const CostModel &cm,
                                          const std::vector<int32_t> &scope) {
  std::vector<int32_t> linalg;
  for (int32_t op : scope)
    if (g.is_linalg(op)) linalg.push_back(op);
  std::unordered_set<int32_t> set(linalg.begin(), linalg.end());
  std::unordered_map<int32_t, int32_t> parent, rank;
  for (int32_t op : linalg) { parent[op] = op; rank[op] = 0; }
  auto find = [&](int32_t x) {
    while (parent[x] != x) { parent[x] = parent[parent[x]]; x = parent[x]; }
    return x;
  };
  auto unite = [&](int32_t a, int32_t b) {
    a = find(a); b = find(b);
    if (a == b) return;
    if (rank[a] < rank[b]) std::swap(a, b);
    parent[b] = a;
    if (rank[a] == rank[b]) ++rank[a];
  };
  for (int32_t consumer : linalg) {
    for (int32_t v : g.ops[consumer].operands) {
      const int32_t p = g.values[v].def;
      if (p < 0 || !set.count(p) || is_reshape_boundary(g, p)) continue;
      bool reshape_between = false;
      for (int32_t u : g.values[v].users)
        if (u != consumer && is_reshape_boundary(g, u)) { reshape_between = true; break; }
      if (reshape_between || !g.has_one_use(p)) continue;
      if (!cm.subgraph_fusion_profitable({p, consumer}).fuse) continue;
      const TileAlignment al = cm.tile_alignment({p, consumer});
      if (!al.aligned && al.overhead_bytes > cm.target().sram_per_core / 4) continue;
      unite(p, consumer);
    }
  }
  std::unordered_map<int32_t, std::vector<int32_t>> by_root;
  std::vector<int32_t> roots;  // in order of each group's first op
  for (int32_t op : linalg) {
    const int32_t r = find(op);
    if (!by_root.count(r)) roots.push_back(r);
    by_root[r].push_back(op);
  }
  std::vector<OutlinedGroup> out;
  for (int32_t r : roots) {
    std::vector<int32_t> ops = by_root[r];
    if (ops.size() <= 1) continue;
    std::sort(ops.begin(), ops.end());  // op ids are block order
    OutlinedGroup grp;
    grp.ops = ops;
    std::unordered_set<int32_t> in_group(ops.begin(), ops.end()), produced, seen;
    for (int32_t op : ops)
      for (int32_t res : g.ops[op].results) produced.insert(res);
    for (int32_t op : ops)
      for (int32_t v : g.ops[op].operands)
        if (!produced.count(v) && seen.insert(v).second) grp.inputs.push_back(v);
    std::unordered_set<int32_t> seen_out;
    for (int32_t op : ops)
      for (int32_t res : g.ops[op].results) {
        bool outside = false;
        for (int32_t u : g.values[res].users)
          if (!in_group.count(u)) { outside = true; break; }
        if (outside && seen_out.insert(res).second) grp.outputs.push_back(res);
      }
    for (int32_t res : g.ops[ops.back()].results)
      if (seen_out.insert(res).second) grp.outputs.push_back(res);
    grp.name = "fused";
    for (int32_t op : ops) grp.name += "_" + short_op_name(g, op);
    grp.name += "_" + std::to_string(out.size());
    out.push_back(std::move(grp));
  }
  return out;
}

bool spatial_decision(const ir::Graph &g, const CostModel &cm, int32_t op, int64_t cores,
                      SpatialDecision *d) {
  const OpKind k = g.ops[op].kind;
  if (!(k == OpKind::Matmul || k == OpKind::BatchMatmul || k == OpKind::Conv2dNchwFchw ||
        k == OpKind::Conv2dNhwcFhwc || k == OpKind::DepthwiseNhwcHwc ||
        k == OpKind::Transpose || k == OpKind::Generic))
    return false;
  if (g.ops[op].results.empty()) return false;
  const ir::Type &out = g.type(g.ops[op].results[0]);
  for (int64_t x : out.shape)
    if (x < 0) return false;
  const size_t loops = num_loops(g, op);
  const OperatorTilingSpec *spec = get_tiling_spec(g, op);
  int32_t best_iter = 0;
  int64_t best_cost = std::numeric_limits<int64_t>::max();
  if (spec) {
    for (const auto &s : spec->split_dims) {
      if (!s.parallel || s.iter_dim >= loops) continue;
      int64_t size = 0;
      if (s.output_dim < out.shape.size()) size = out.shape[s.output_dim];
      if (size <= 1) continue;
      const SpatialSplitCost c = cm.spatial_split_detailed(op, s, cores);
      d->candidates.push_back({(int32_t)s.iter_dim, c.total_cycles});
      if (c.total_cycles < best_cost) { best_cost = c.total_cycles; best_iter = (int32_t)s.iter_dim; }
    }
  } else {
    const auto &it = g.ops[op].iters;
    for (unsigned od = 0; od < out.shape.size(); ++od) {
      if (od >= loops || (od < it.size() && it[od] != 0)) continue;
      const ScheduleCost c = cm.spatial_split(op, od, cores);
      d->candidates.push_back({(int32_t)od, c.total_cycles});
      if (c.total_cycles < best_cost) { best_cost = c.total_cycles; best_iter = (int32_t)od; }
    }
  }
  int32_t best_out = best_iter;
  if (spec)
    for (const auto &s : spec->split_dims)
      if ((int32_t)s.iter_dim == best_iter) {
        if (s.output_dim < out.shape.size()) best_out = (int32_t)s.output_dim;
        break;
      }
  d->iter_dim = best_iter;
  d->out_dim = best_out;
  d->dim_size = out.shape[best_out];
  d->tile_size = (d->dim_size + cores - 1) / cores;
  d->full_iters = d->dim_size / d->tile_size;
  d->peel_size = d->dim_size - d->full_iters * d->tile_size;
  d->cost = best_cost;
  return true;
}

namespace {

// TemporalTilingPass.cpp:76-254
TileConfig spec_driven_search(const ir::Graph &g, const CostModel &cm, int32_t op,
                              const OperatorTilingSpec &spec) {
  TileConfig best;
  best.cost = {0, 0, kInf, 0, 0, 0};
  const ir::Op &o = g.ops[op];
  if (o.results.empty()) return best;
  const ir::Type &out = g.type(o.results[0]);
  const std::vector<int64_t> sizes = iter_sizes(g, op);
  const size_t loops = sizes.size();
  std::vector<std::pair<uint32_t, std::vector<int64_t>>> cands;
  for (uint32_t pref : spec.preferred_temporal_dims) {
    if (pref >= spec.split_dims.size()) continue;
    const uint32_t d = spec.split_dims[pref].iter_dim;
    if (d >= loops || sizes[d] <= 0) continue;
    cands.push_back({d, CostModel::tile_candidates(sizes[d])});
  }
  if (cands.empty()) return best;
  const int64_t dtb = std::max<int64_t>(1, out.bits / 8);
  auto for_dim = [&](uint32_t d, int64_t full) {
    for (const auto &[dim, c] : cands)
      if (dim == d) return c;
    return std::vector<int64_t>{full};
  };
  if (o.kind == OpKind::Matmul) {
    const int64_t M = out.shape[0], N = out.shape[1], K = g.type(o.operands[0]).shape[1];
    for (int64_t tm : for_dim(0, M))
      for (int64_t tn : for_dim(1, N))
        for (int64_t tk : for_dim(2, K)) {
          const ScheduleCost c = cm.matmul_tile(tm, tn, tk, M, N, K, dtb);
          if (c.total_cycles < best.cost.total_cycles) {
            best.tile_sizes.assign(loops, 0);
            best.tile_sizes[0] = tm; best.tile_sizes[1] = tn; best.tile_sizes[2] = tk;
            best.cost = c;
          }
        }
    return best;
  }
  if (o.kind == OpKind::Conv2dNchwFchw) {
    const ir::Type &in = g.type(o.operands[0]), &f = g.type(o.operands[1]);
    const int64_t N_ = out.shape[0], Co = out.shape[1], Ho = out.shape[2], Wo = out.shape[3];
    const int64_t Ci = in.shape[1], Kh = f.shape[2], Kw = f.shape[3];
    for (int64_t tn : for_dim(0, N_))
      for (int64_t tco : for_dim(1, Co))
        for (int64_t th : for_dim(2, Ho))
          for (int64_t tw : for_dim(3, Wo)) {
            const ScheduleCost c = cm.conv2d_tile(tn, tco, th, tw, N_, Co, Ho, Wo, Ci, Kh, Kw, {1, 1}, dtb);
            if (c.total_cycles < best.cost.total_cycles) {
              best.tile_sizes.assign(loops, 0);
              best.tile_sizes[0] = tn; best.tile_sizes[1] = tco;
              best.tile_sizes[2] = th; best.tile_sizes[3] = tw;
              best.cost = c;
            }
          }
    return best;
  }
  if (o.kind == OpKind::Conv2dNhwcFhwc) {  // iteration order (n, oh, ow, f, kh, kw, c)
    const ir::Type &in = g.type(o.operands[0]), &f = g.type(o.operands[1]);
    const int64_t N_ = out.shape[0], Ho = out.shape[1], Wo = out.shape[2], Co = out.shape[3];
    const int64_t Ci = in.shape[3], Kh = f.shape[1], Kw = f.shape[2];
    for (int64_t tn : for_dim(0, N_))
      for (int64_t th : for_dim(1, Ho))
        for (int64_t tw : for_dim(2, Wo))
          for (int64_t tco : for_dim(3, Co)) {
            const ScheduleCost c = cm.conv2d_tile(tn, tco, th, tw, N_, Co, Ho, Wo, Ci, Kh, Kw, {1, 1}, dtb);
            if (c.total_cycles < best.cost.total_cycles) {
              best.tile_sizes.assign(loops, 0);
              best.tile_sizes[0] = tn; best.tile_sizes[1] = th;
              best.tile_sizes[2] = tw; best.tile_sizes[3] = tco;
              best.cost = c;
            }
          }
    return best;
  }
  if (o.kind == OpKind::Generic) {
    const uint32_t td_dim = cands[0].first;
    const int64_t size = sizes[td_dim];
    int64_t per_row = 1;
    for (size_t i = 0; i < out.shape.size(); ++i)
      if (i != td_dim) per_row *= out.shape[i];
    const int64_t bytes_per_row = per_row * dtb * 3;
    for (int64_t td : cands[0].second) {
      const int64_t sram = td * bytes_per_row * 2;
      if (sram > cm.target().sram_per_core) continue;
      const int64_t tiles = (size + td - 1) / td;
      const int64_t comp = std::max<int64_t>(1, (td * per_row) / cm.target().dsp_throughput);
      const int64_t dma = cm.dma_cycles(td * bytes_per_row);
      const int64_t total = tiles <= 1 ? dma + comp + dma
                                       : dma + (tiles - 1) * std::max(dma, comp) + comp + dma;
      if (total < best.cost.total_cycles) {
        best.tile_sizes.assign(loops, 0);
        best.tile_sizes[td_dim] = td;
        best.cost = {tiles * comp, tiles * dma * 2, total, sram, tiles, tiles * td * bytes_per_row * 2};
      }
    }
  }
  return best;
}

}  // namespace

bool temporal_decision(const ir::Graph &g, const CostModel &cm, int32_t op, TileConfig *out) {
  const OpKind k = g.ops[op].kind;
  if (!(k == OpKind::Matmul || k == OpKind::BatchMatmul || k == OpKind::Conv2dNchwFchw ||
        k == OpKind::Conv2dNhwcFhwc || k == OpKind::Transpose || k == OpKind::Generic))
    return false;
  TileConfig c;
  c.cost = {0, 0, kInf, 0, 0, 0};
  const OperatorTilingSpec *spec = get_tiling_spec(g, op);
  if (spec && !spec->preferred_temporal_dims.empty()) c = spec_driven_search(g, cm, op, *spec);
  if (c.tile_sizes.empty() || !c.cost.valid()) c = cm.best_tile_config(op);
  if (c.tile_sizes.empty() || !c.cost.valid() || c.cost.num_tiles <= 1) return false;
  if (g.ops[op].results.empty()) return false;
  const size_t loops = num_loops(g, op);
  c.tile_sizes.resize(loops, 0);
  *out = c;
  return true;
}

std::vector<BarrierAssignment> barrier_alloc(const std::vector<SchedKind> &ops, int64_t pool) {
  std::vector<BarrierAssignment> out(ops.size());
  int64_t sub = -1;
  bool open = false;  // the current subgraph holds an op
  SchedKind prev = SchedKind::Ignore;
  for (size_t i = 0; i < ops.size(); ++i) {
    const SchedKind k = ops[i];
    if (k == SchedKind::Ignore) continue;
    const bool cut = k == SchedKind::DmaIn && (prev == SchedKind::DmaOut || prev == SchedKind::Compute);
    if (!open || (cut && open)) {
      ++sub;
      open = true;
    }
    out[i].subgraph = sub;
    out[i].barrier_id = sub % pool;
    out[i].generation = sub / pool;
    prev = k;
  }
  return out;
}

}  // namespace npu

