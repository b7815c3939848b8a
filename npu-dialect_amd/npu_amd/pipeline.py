"""The decision pipeline in the reference's pass order, MLIR-free.

``npu-pipeline`` (lib/Transforms/Pipeline.cpp:11-38; the harness variant
tools/harness/run_pipeline.py:25-36) runs, per module:

    npu-fusion -> npu-outline-fused-groups -> npu-spatial-tiling ->
    npu-core-mapping -> npu-temporal-tiling -> canonicalize/cse ->
    npu-bufferize -> npu-sram-allocation -> npu-barrier-alloc ->
    npu-cost-evaluate

``run`` replays those decisions on one parsed function with the host
library (libnpu_host.so) and returns them as data: the fusion groups, the
outlined functions (name, signature), each function's spatial and temporal
tile decisions, its DMA/SRAM plan and its COST_JSON record, and -- for the
MI355X -- the entry point that executes the outlined group.  Canonicalize/CSE
only fold the constants peeling leaves behind, so they have no decision to
restate; barrier allocation cuts a tile loop's DMA and compute ops into
subgraphs, which ``tileplan`` applies to one tile loop (host.barrier_alloc)
next to the loop's SRAM plan at its slice sizes.  Core mapping tags each spatial tile with its core
id, (iv - lb) / step (CoreMappingPass.cpp:33-73); on the GPU that is the
workgroup index, so the report gives the core (CU) count of each tiled op.

Where the reference walks the outlined functions as separate FuncOps, this
works on the group's op list within the one parsed function (the outlined
body is exactly those ops).
"""
from __future__ import annotations

from . import host, mlir

# outlined op chain (index stripped) -> MI355X entry point
from .names import OUTLINED_NAMES

STEPS = ("fusion", "outline", "spatial", "core-map", "temporal", "canonicalize", "bufferize",
         "sram-alloc", "barrier-alloc", "cost-eval")


def _chain(name: str) -> str:
    return name.rsplit("_", 1)[0]


def _tiles(sizes):
    n = 1
    for d, t in sizes:
        if t and t > 0:
            n *= -(-d // t)
    return n


def run(func: mlir.MFunc, target: host.HWTarget = None, cores: int = None,
        sram_size: int = None, fresh: bool = True) -> dict:
    """Replays npu-pipeline's decisions on `func`; see the module docstring.
    The target is `target` when given, else the module's #npu.target (as
    CostModelAnalysis reads it, lib/Analysis/CostModel.cpp:985-1000), else
    the reference's default NPU.  `fresh`: decide as a new npu-opt process
    would (the conv tiling spec is rebuilt from this function's first conv);
    False keeps the spec of the functions run before (later functions of one
    module)."""
    if fresh:
        host.spec_reset()
    if target is not None:
        t = target
    elif func.target:
        t = host.target_from_params(func.target)
    else:
        t = host.default_target()
    cores = cores or t.num_cores
    sram = sram_size or t.sram_per_core
    g = host.Graph(func)
    names = {v: k for k, v in g.value_id.items()}
    ops = func.ops
    rep = {"function": func.name, "steps": list(STEPS), "target": t.as_dict()}

    rep["fusion_groups"] = [[ops[i].results[0] if ops[i].results else ops[i].name for i in grp]
                            for grp in host.fusion_groups(g, t)]
    outlined = host.outline_groups(g, t)
    grouped = {i for grp in outlined for i in grp["ops"]}
    funcs = [{"name": grp["name"], "ops": grp["ops"], "inputs": grp["inputs"],
              "outputs": grp["outputs"],
              "entry_point": OUTLINED_NAMES.get(_chain(grp["name"]))} for grp in outlined]
    parent = [i for i in g.linalg_ops() if i not in grouped]
    if parent:
        funcs.append({"name": func.name, "ops": parent, "inputs": [], "outputs": [],
                      "entry_point": None})

    cost_lines = []
    for f in funcs:
        # spatial tiling and core mapping of each linalg op of the function
        sp = []
        for i in f["ops"]:
            d = host.spatial(g, t, i, cores)
            if d is not None:
                sp.append({"op": ops[i].results[0] if ops[i].results else ops[i].name,
                           "iter_dim": d.iter_dim, "tile": d.tile_size, "full_iters": d.full_iters,
                           "peel": d.peel_size, "cores": cores,
                           "candidates": [list(c) for c in d.candidates]})
        f["spatial"] = sp
        # temporal tiling: the spec-driven tile of each matrix op
        tp, trips = [], 1
        for i in f["ops"]:
            ts, cost = host.temporal(g, t, i)
            if ts is not None:
                tp.append({"op": ops[i].results[0] if ops[i].results else ops[i].name,
                           "tiles": ts, "num_tiles": cost.num_tiles,
                           "total_cycles": cost.total_cycles})
                trips = max(trips, cost.num_tiles)
        f["temporal"] = tp
        # bufferize + SRAM plan of the function's tile loop, then its cost record
        bufs = host.bufferize(g, f["ops"])
        summ = host.sram_allocation(bufs, sram)
        f["sram"] = {"buffers": [{"value": names.get(b.value, str(b.value)),
                                  "role": host.ROLES[b.role], "bytes": b.bytes,
                                  "offset": b.addr, "offset_pong": b.addr_pong,
                                  "double_buffered": bool(b.double_buffered),
                                  "prefetch_addr": b.prefetch_addr, "spilled": bool(b.spilled)}
                                 for b in bufs],
                     "spilled": summ.spilled, "prefetched": summ.prefetched,
                     "peak_bytes": summ.peak_bytes}
        kc = host.cost_evaluate(g, t, f["ops"], bufs, trips)
        f["cost"] = kc
        cost_lines.append(host.cost_json(f["name"], kc))
    rep["functions"] = funcs
    rep["cost_json"] = cost_lines
    return rep


def run_file(path: str, target: host.HWTarget = None, **kw) -> list:
    """`run` on every function of an .mlir file, as one npu-opt process."""
    return [run(f, target, fresh=i == 0, **kw) for i, f in enumerate(mlir.parse_file(path))]
