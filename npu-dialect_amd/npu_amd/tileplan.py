"""The reference's memory plan of a tile loop, as the LDS layout of a launch.

For the group ``fill -> matmul -> generic(bias add, act)``, the reference's
npu-temporal-tiling picks a tile (tm, tn, tk) for the matmul
(TemporalTilingPass.cpp:76-336); npu-bufferize gives every slice the tile
loop uses an SRAM buffer of the slice's size (BufferizePass.cpp:97-222);
npu-sram-allocation places those buffers with its dual-end allocator, the
loop's inputs in ping/pong pairs (SRAMAllocationPass.cpp:172-342); and
npu-barrier-alloc cuts the loop's DMA-in -> compute -> DMA-out ops into
subgraphs with barrier ids and generations (DMASchedulingPass.cpp:92-147).

``matmul_group_plan`` replays those decisions with the host library at the
MI355X target, whose SRAM is one CU's LDS (163 840 bytes), and returns the
``npu_tile_plan`` that ``groups.planned_matmul_bias_act`` launches with:
each buffer at its planned byte offset in the workgroup's LDS.
"""
from __future__ import annotations

from . import _lib, host, mlir, pipeline

LDS_BYTES = 163840


def _group_values(func, ops):
    """Names of the group's slices: A, B (matmul ins), init (fill outs), bias
    (the generic's other input), y (the generic's outs)."""
    by = {func.ops[i].name: func.ops[i] for i in ops}
    fill, mm, gen = by.get("linalg.fill"), by.get("linalg.matmul"), by.get("linalg.generic")
    if mm is None or gen is None:
        raise NotImplementedError("the tile plan covers fill -> matmul -> generic groups")
    mm_out = mm.results[0]
    bias = [v for v in gen.ins if v != mm_out]
    return {"A": mm.ins[0], "B": mm.ins[1], "init": (fill.outs[0] if fill else mm.outs[0]),
            "bias": bias[0] if bias else None, "y": gen.outs[0]}


def matmul_group_plan(func: mlir.MFunc, target: host.HWTarget = None, sram: int = LDS_BYTES,
                      pool: int = 4) -> dict:
    """The fill -> matmul -> generic group of `func`: its temporal tile, the
    tile loop's buffers planned at `sram` bytes, the barrier allocation of
    one loop trip, and the npu_tile_plan of a launch with that layout."""
    t = target or host.mi355x_target(32)
    rep = pipeline.run(func, t, sram_size=sram)
    f = next((f for f in rep["functions"] if f["entry_point"] == "fused_matmul_bias_act"), None)
    if f is None:
        raise NotImplementedError("no fill -> matmul -> generic group in this function")
    mm_i = next(i for i in f["ops"] if func.ops[i].name == "linalg.matmul")
    mm_res = func.ops[mm_i].results[0]
    tiles = next(d["tiles"] for d in f["temporal"] if d["op"] == mm_res)
    tm, tn, tk = tiles[:3]
    names = _group_values(func, f["ops"])
    elem = 4  # f32 (f16 text runs as f32, the reference harness's rule)
    slice_bytes = {names["A"]: tm * tk * elem, names["B"]: tk * tn * elem,
                   names["init"]: tm * tn * elem, names["y"]: tm * tn * elem}
    if names["bias"]:
        slice_bytes[names["bias"]] = tn * elem
    g = host.Graph(func)
    bufs = host.bufferize(g, f["ops"], slice_bytes)
    summ = host.sram_allocation(bufs, sram)
    vname = {v: k for k, v in g.value_id.items()}
    planned = {vname.get(b.value, str(b.value)): b for b in bufs}
    layout = {}
    for key in ("A", "B", "bias", "init", "y"):
        b = planned.get(names[key]) if names[key] else None
        if b is None:
            continue
        if b.spilled:
            raise NotImplementedError(f"the plan spills {names[key]} to DRAM")
        layout[key] = {"value": names[key], "bytes": b.bytes, "offset": b.addr,
                       "offset_pong": b.addr_pong, "double_buffered": bool(b.double_buffered),
                       "role": host.ROLES[b.role]}
    # one trip of the bufferized tile loop: the DMAs into SRAM, the compute
    # ops, the DMA out (the output slice), for every K step
    nk = -(-func.types[names["A"]].shape[1] // tk)
    trip = ["dma_in"] * (3 if names["bias"] else 2) + ["compute"] * 3 + ["dma_out"]
    barriers = host.barrier_alloc(trip * nk, pool)
    for key in ("A", "B"):
        if not layout[key]["double_buffered"]:
            # the launch fetches K step i + 1 into the other buffer while
            # step i is multiplied: it needs both halves of the pair
            raise NotImplementedError(f"the plan gives {key} no ping/pong pair at {sram} bytes")
    plan = _lib.NpuTilePlan()
    plan.tm, plan.tn, plan.tk, plan.lds_bytes = tm, tn, tk, sram
    plan.off_a, plan.off_a_pong = layout["A"]["offset"], layout["A"]["offset_pong"]
    plan.off_b, plan.off_b_pong = layout["B"]["offset"], layout["B"]["offset_pong"]
    plan.off_bias = layout["bias"]["offset"] if "bias" in layout else -1
    plan.off_c, plan.off_y = layout["init"]["offset"], layout["y"]["offset"]
    return {"function": f["name"], "tile": (tm, tn, tk), "k_steps": nk, "buffers": layout,
            "peak_bytes": summ.peak_bytes, "barriers": barriers,
            "subgraphs": max(s for s, _, _ in barriers) + 1, "plan": plan}
