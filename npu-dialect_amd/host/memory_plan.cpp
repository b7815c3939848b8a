// memory_plan.cpp -- DMA insertion, the dual-end SRAM plan and the
// per-function cost record (see memory_plan.hpp).
#include "memory_plan.hpp"

#include <algorithm>
#include <numeric>

namespace npu {

// ------------------------------------------------ SRAMAllocationPass.cpp:127-162
int64_t DualEndAllocator::alloc_low(int64_t b) {
  const int64_t a = align(b);
  if (low + a > high) return -1;
  const int64_t addr = low;
  low += a;
  return addr;
}

int64_t DualEndAllocator::alloc_high(int64_t b) {
  const int64_t a = align(b);
  if (high - a < low) return -1;
  high -= a;
  return high;
}

void DualEndAllocator::free_low(int64_t b) {
  low -= align(b);
  if (low < 0) low = 0;
}

// ------------------------------------------------ SRAMAllocationPass.cpp:172-342
SramPlanSummary plan_sram(std::vector<SramBuffer> &bufs, int64_t sram_size) {
  SramPlanSummary sum;
  if (bufs.empty()) return sum;
  DualEndAllocator alloc(sram_size);

  // phase 1: liveness-aware dual-end allocation, in first-use order
  std::vector<size_t> order(bufs.size());
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(),
                   [&](size_t a, size_t b) { return bufs[a].first_use < bufs[b].first_use; });
  std::vector<std::pair<size_t, int64_t>> active;  // (buffer, last use)
  std::vector<size_t> spill;
  for (size_t idx : order) {
    SramBuffer &buf = bufs[idx];
    // release buffers dead before this one's first use (outputs stay: they
    // are written back at the end); the low end shrinks by their size
    std::vector<std::pair<size_t, int64_t>> still;
    for (const auto &a : active) {
      if (a.second < buf.first_use) {
        const SramBuffer &d = bufs[a.first];
        if (d.role != BufRole::Output) {
          alloc.free_low(d.bytes);
          if (d.double_buffered) alloc.free_low(d.bytes);
        }
      } else {
        still.push_back(a);
      }
    }
    active = std::move(still);

    bool want_db = buf.role == BufRole::Input && buf.in_loop;
    int64_t addr = -1, pong = -1;
    switch (buf.role) {
      case BufRole::Input:
        addr = alloc.alloc_low(buf.bytes);
        if (addr >= 0 && want_db) {
          pong = alloc.alloc_low(buf.bytes);
          if (pong < 0) want_db = false;  // no room for the pong copy
        }
        break;
      case BufRole::Output:
        addr = alloc.alloc_high(buf.bytes);
        break;
      case BufRole::Intermediate:
        addr = alloc.alloc_middle(buf.bytes);
        break;
    }
    if (addr >= 0) {
      buf.addr = addr;
      buf.double_buffered = want_db;
      if (want_db) buf.addr_pong = pong;
      active.push_back({idx, buf.last_use});
    } else {
      spill.push_back(idx);
    }
  }
  // phase 2: what did not fit lives in DRAM
  for (size_t idx : spill) bufs[idx].spilled = true;
  sum.spilled = (int64_t)spill.size();

  // phase 4: prefetch of the next tile's inputs into the space left, largest
  // first, from the high end
  const int64_t free_after = alloc.free_bytes();
  sum.free_after = free_after;
  if (free_after > 0) {
    std::vector<size_t> cand;
    for (size_t i = 0; i < bufs.size(); ++i)
      if (!bufs[i].spilled && bufs[i].addr >= 0 && bufs[i].role == BufRole::Input) cand.push_back(i);
    std::stable_sort(cand.begin(), cand.end(),
                     [&](size_t a, size_t b) { return bufs[a].bytes > bufs[b].bytes; });
    int64_t budget = free_after;
    for (size_t i : cand) {
      if (bufs[i].bytes > budget) continue;
      const int64_t pa = alloc.alloc_high(bufs[i].bytes);
      if (pa < 0) continue;
      bufs[i].prefetch_addr = pa;
      budget -= DualEndAllocator::align(bufs[i].bytes);
      ++sum.prefetched;
    }
    sum.prefetch_bytes = free_after - budget;
  }
  for (const SramBuffer &b : bufs)
    if (!b.spilled && b.addr >= 0) {
      sum.peak_bytes = std::max(sum.peak_bytes, b.addr + b.bytes);
      if (b.addr_pong >= 0) sum.peak_bytes = std::max(sum.peak_bytes, b.addr_pong + b.bytes);
    }
  return sum;
}

// ------------------------------------------------ BufferizePass.cpp:97-222
std::vector<SramBuffer> bufferize_loop(const ir::Graph &g, const std::vector<int32_t> &ops,
                                       const std::vector<int64_t> *bytes) {
  std::vector<char> inside(g.ops.size(), 0);
  for (int32_t o : ops) inside[o] = 1;
  std::vector<int32_t> dram;     // defined outside, used inside: first-use order
  std::vector<char> written(g.values.size(), 0);
  std::vector<int64_t> last_op(g.values.size(), -1);
  for (size_t j = 0; j < ops.size(); ++j) {
    const ir::Op &op = g.ops[ops[j]];
    if (op.kind == ir::OpKind::Return) continue;
    for (size_t k = 0; k < op.operands.size(); ++k) {
      const int32_t v = op.operands[k];
      const ir::Value &val = g.values[v];
      if (!val.type.shaped) continue;                        // only memrefs
      if (val.def >= 0 && inside[val.def]) continue;         // defined in the loop
      if (val.def >= 0 && g.ops[val.def].kind == ir::OpKind::Constant) continue;
      if (std::find(dram.begin(), dram.end(), v) == dram.end()) dram.push_back(v);
      if (g.is_linalg(ops[j]) && (int32_t)k >= op.num_inputs) written[v] = 1;  // a DPS init
      last_op[v] = (int64_t)j;
    }
  }
  // program steps: [alloc_sram, dma_copy] per buffer, the ops, the copies back
  const int64_t n = (int64_t)dram.size();
  std::vector<SramBuffer> bufs;
  int64_t back = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int32_t v = dram[i];
    SramBuffer b;
    b.value = v;
    b.bytes = bytes && (size_t)v < bytes->size() && (*bytes)[v] > 0 ? (*bytes)[v]
                                                                     : CostModel::tensor_bytes(g.type(v));
    b.role = written[v] ? BufRole::Output : BufRole::Input;
    b.first_use = 2 * i;
    b.last_use = std::max<int64_t>(2 * i + 1, 2 * n + last_op[v]);
    if (written[v]) b.last_use = 2 * n + (int64_t)ops.size() + back++;
    b.in_loop = true;
    bufs.push_back(b);
  }
  return bufs;
}

// ------------------------------------------------ CostEvaluatePass.cpp:57-168
KernelCost cost_evaluate(const ir::Graph &g, const CostModel &cm, const std::vector<int32_t> &ops,
                         const std::vector<SramBuffer> &bufs, int64_t tile_iterations) {
  KernelCost kc;
  std::vector<int32_t> lin;
  for (int32_t o : ops)
    if (g.is_linalg(o)) lin.push_back(o);
  kc.num_linalg_ops = (int64_t)lin.size();
  if (!lin.empty()) {
    const RooflineCost rc = cm.roofline(lin);
    kc.flops = rc.flops;
    kc.mem_bytes = rc.mem_bytes;
    kc.arithmetic_intensity = rc.arithmetic_intensity;
    kc.time_sec = rc.time_sec;
    kc.memory_bound = rc.memory_bound;
    kc.efficiency = rc.efficiency;
  }
  for (const SramBuffer &b : bufs) {
    kc.dma_in_bytes += b.bytes;  // every buffer is filled by a DRAM->SRAM copy
    if (b.role == BufRole::Output) kc.dma_out_bytes += b.bytes;
  }
  for (int32_t o : lin) {
    const int64_t c = cm.compute_cycles(o);
    if (cm.is_matrix_op(o))
      kc.matrix_cycles += c;
    else
      kc.dsp_cycles += c;
  }
  for (const SramBuffer &b : bufs)
    if (!b.spilled && b.addr >= 0) kc.peak_sram_bytes = std::max(kc.peak_sram_bytes, b.addr + b.bytes);
  kc.num_tile_iterations = tile_iterations;
  kc.sram_budget = cm.target().sram_per_core;
  return kc;
}

}  // namespace npu
