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


def _conv_group(func, f):
    by = {func.ops[i].name: func.ops[i] for i in f["ops"]}
    fill, conv = by.get("linalg.fill"), by.get("linalg.conv_2d_nchw_fchw")
    gen = by.get("linalg.generic")
    if conv is None or gen is None:
        raise NotImplementedError("the conv tile plan covers fill -> conv_2d_nchw_fchw -> generic "
                                  "groups")
    bias = [v for v in gen.ins if v != conv.results[0]]
    return conv, {"x": conv.ins[0], "w": conv.ins[1],
                  "init": fill.outs[0] if fill else conv.outs[0],
                  "bias": bias[0] if bias else None, "y": gen.outs[0]}


def conv_group_plan(func: mlir.MFunc, target: host.HWTarget = None, cores: int = 256,
                    sram: int = LDS_BYTES) -> dict:
    """The fill -> conv_2d_nchw_fchw -> generic group of `func` (its input the
    padded tensor) as `npu-opt --npu-spatial-tiling=num-cores=<cores>
    --npu-temporal-tiling=sram-size=<sram> --npu-bufferize
    --npu-sram-allocation=sram-size=<sram>` plans it: the spatial split of the
    conv over output rows (one row per core: SpatialTilingPass.cpp:38-168),
    the spec-driven temporal tile of a core's row over output channels
    (TemporalTilingPass.cpp:76-336), the loop's slice buffers placed by the
    dual-end allocator -- ping/pong for inputs in the loop, the weight
    prefetch into the SRAM left over, spills to DRAM
    (SRAMAllocationPass.cpp:172-363).  Returns the plan, the buffers and the
    npu_conv_tile_plan a launch uses (-1 for a buffer the plan does not put in
    SRAM).  `target`: the module's, else the reference's default."""
    import copy
    t = target or (host.target_from_params(func.target) if func.target else host.default_target())
    rep = pipeline.run(func, t, cores=cores, sram_size=sram)
    f = next((f for f in rep["functions"]
              if any(func.ops[i].name == "linalg.conv_2d_nchw_fchw" for i in f["ops"])), None)
    if f is None:
        raise NotImplementedError("no conv_2d_nchw_fchw group in this function")
    conv, names = _conv_group(func, f)
    if conv.attrs.get("strides", [1, 1]) != [1, 1]:
        raise NotImplementedError(f"{conv.results[0]}: strides {conv.attrs['strides']}")
    N, C, Hp, Wp = func.types[names["x"]].shape
    F, _, KH, KW = func.types[names["w"]].shape
    Ho, Wo = Hp - KH + 1, Wp - KW + 1
    sp = next((d for d in f["spatial"] if d["op"] == conv.results[0]), None)
    if sp is None or sp["iter_dim"] != 2 or sp["tile"] != 1:
        raise NotImplementedError(f"{conv.results[0]}: the spatial split is {sp}, not one output "
                                  "row per core")
    # one core's share: output row [1, F, 1, Wo] from input rows [1, C, KH, Wp]
    share = (f"func.func @row(%x: tensor<1x{C}x{KH}x{Wp}xf32>, %w: tensor<{F}x{C}x{KH}x{KW}xf32>, "
             f"%o: tensor<1x{F}x1x{Wo}xf32>) -> tensor<1x{F}x1x{Wo}xf32> {{\n"
             f"  %r = linalg.conv_2d_nchw_fchw {{dilations = dense<1> : tensor<2xi64>, strides = "
             f"dense<1> : tensor<2xi64>}} ins(%x, %w : tensor<1x{C}x{KH}x{Wp}xf32>, "
             f"tensor<{F}x{C}x{KH}x{KW}xf32>) outs(%o : tensor<1x{F}x1x{Wo}xf32>) -> "
             f"tensor<1x{F}x1x{Wo}xf32>\n  return %r : tensor<1x{F}x1x{Wo}xf32>\n}}\n")
    t2 = copy.copy(t)
    t2.sram_per_core = sram
    ts, _ = host.temporal(host.Graph(mlir.parse_functions(share)[0]), t2, 0)
    if ts is None:
        # one tile (TemporalTilingPass leaves an op whose best tile count is 1
        # untiled): the core's whole row in one trip
        ts = [1, F, 1, Wo, 0, 0, 0]
    if ts[0] != 1 or ts[2] != 1 or ts[3] != Wo:
        raise NotImplementedError(f"the temporal tile of a row is {ts}, not output-channel tiles")
    tco = min(ts[1], F)
    elem = 4  # f32 (f16 text runs as f32, the reference harness's rule)
    slice_bytes = {names["x"]: C * KH * Wp * elem, names["w"]: tco * C * KH * KW * elem,
                   names["init"]: tco * Wo * elem, names["y"]: tco * Wo * elem}
    if names["bias"]:
        slice_bytes[names["bias"]] = tco * elem
    g = host.Graph(func)
    bufs = host.bufferize(g, f["ops"], slice_bytes)
    summ = host.sram_allocation(bufs, sram)
    vname = {v: k for k, v in g.value_id.items()}
    planned = {vname.get(b.value, str(b.value)): b for b in bufs}
    layout = {}
    for key in ("x", "w", "bias", "init", "y"):
        b = planned.get(names[key]) if names[key] else None
        if b is None:
            continue
        if b.spilled and key not in ("x", "w"):
            raise NotImplementedError(f"the plan spills {names[key]} to DRAM")
        layout[key] = {"value": names[key], "bytes": b.bytes, "spilled": bool(b.spilled),
                       "offset": -1 if b.spilled else b.addr,
                       "offset_pong": b.addr_pong if b.double_buffered and not b.spilled else -1,
                       "double_buffered": bool(b.double_buffered) and not b.spilled,
                       "prefetch_addr": b.prefetch_addr if not b.spilled else -1,
                       "role": host.ROLES[b.role]}
    plan = _lib.NpuConvTilePlan()
    plan.tco, plan.lds_bytes = tco, sram
    plan.off_in, plan.off_in_pong = layout["x"]["offset"], layout["x"]["offset_pong"]
    plan.off_in_prefetch = layout["x"]["prefetch_addr"]
    plan.off_w, plan.off_w_pong = layout["w"]["offset"], layout["w"]["offset_pong"]
    plan.off_w_prefetch = layout["w"]["prefetch_addr"]
    nob = {"offset": -1, "offset_pong": -1, "prefetch_addr": -1}
    bl = layout.get("bias", nob)
    plan.off_bias, plan.off_bias_pong = bl["offset"], bl["offset_pong"]
    plan.off_bias_prefetch = bl["prefetch_addr"]
    plan.off_c, plan.off_y = layout["init"]["offset"], layout["y"]["offset"]
    return {"function": f["name"], "share": (1, F, 1, Wo), "tile": list(ts), "tco": tco,
            "tiles": -(-F // tco), "cores": N * Ho, "buffers": layout,
            "peak_bytes": summ.peak_bytes, "prefetched": summ.prefetched, "plan": plan}
