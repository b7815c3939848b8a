"""The reference's memory plan as a launch's LDS layout (CPU side):
npu-barrier-alloc's subgraphs and barrier ids (DMASchedulingPass.cpp:92-147),
the tile loop's buffers of the fill -> matmul -> generic group planned at one
CU's LDS (163 840 bytes) by the dual-end allocator, and the checks the
plan-driven entry point makes before any launch."""
import ctypes as C

import pytest

import npu_amd
import reference_inputs
from npu_amd import _lib, blocks, configs, host, lower, mlir, tileplan
from npu_amd.memref import F32

from test_abi import _err, _mr


def test_barrier_alloc_cuts_and_numbers_subgraphs():
    # DMA-in after compute or DMA-out starts a subgraph; DMA-ins in a row and
    # a DMA-out after compute stay in it; ids cycle over the pool, the
    # generation counts the cycles; ignored ops get -1
    k = ["dma_in", "dma_in", "compute", "dma_out"] * 5 + ["ignore", "compute", "dma_in"]
    a = host.barrier_alloc(k, 4)
    subs = [s for s, _, _ in a]
    assert subs[:20] == [i // 4 for i in range(20)]
    assert a[20] == (-1, -1, -1)
    assert a[21] == (4, 0, 1)         # compute after DMA-out: same subgraph
    assert a[22] == (5, 1, 1)         # DMA-in after compute: a new one
    assert [a[4 * i][1:] for i in range(5)] == [(0, 0), (1, 0), (2, 0), (3, 0), (0, 1)]
    # a leading compute opens the first subgraph; pool 1 makes every
    # subgraph its own generation
    assert [x[2] for x in host.barrier_alloc(["compute", "dma_in", "compute"], 1)] == [0, 1, 1]
    assert host.barrier_alloc([], 4) == []
    with pytest.raises(Exception):
        host.barrier_alloc(["dma_in"], 0)


def test_c1_group_plan_at_the_lds_size():
    """The C1 group at the MI355X target: temporal tile (128, 64, 16), the
    tile loop's slices planned at 163 840 bytes.  By the allocator's rules:
    inputs from the low end in first-use order, each pong right after its
    ping (64-byte aligned); outputs from the high end in first-use order."""
    f = mlir.parse_functions(configs.linalg_text(configs.matmul_bias_relu()))[0]
    p = tileplan.matmul_group_plan(f)
    assert p["tile"] == (128, 64, 16) and p["k_steps"] == 512 // 16
    b = p["buffers"]
    A, B, bias = 128 * 16 * 4, 16 * 64 * 4, 64 * 4
    assert (b["A"]["offset"], b["A"]["offset_pong"]) == (0, A)
    assert (b["B"]["offset"], b["B"]["offset_pong"]) == (2 * A, 2 * A + B)
    assert (b["bias"]["offset"], b["bias"]["offset_pong"]) == (2 * A + 2 * B, 2 * A + 2 * B + bias)
    tile = 128 * 64 * 4
    assert b["init"]["offset"] == 163840 - tile and b["y"]["offset"] == 163840 - 2 * tile
    # the simulator's bound (offset + size <= SRAM) and no overlaps
    spans = []
    for v in b.values():
        for off in (v["offset"], v["offset_pong"]):
            if off >= 0:
                assert off + v["bytes"] <= 163840
                spans.append((off, off + v["bytes"]))
    spans.sort()
    assert all(e <= s for (_, e), (s, _) in zip(spans, spans[1:]))
    # one subgraph per K step: DMA-ins, the three compute ops, the copy back
    assert p["subgraphs"] == 32
    assert p["barriers"][7 * 5][1:] == (1, 1)  # K step 5: barrier 1, generation 1
    plan = p["plan"]
    assert (plan.tm, plan.tn, plan.tk, plan.lds_bytes) == (128, 64, 16, 163840)
    assert (plan.off_c, plan.off_y, plan.off_bias) == (b["init"]["offset"], b["y"]["offset"],
                                                       b["bias"]["offset"])


@pytest.mark.skipif(not reference_inputs.available(), reason="the reference's test inputs")
def test_matmul_relu_group_plan():
    """test/matmul_relu.mlir (f16 text, run as f32 by the harness rule): no
    bias buffer, the plan has none."""
    f = mlir.parse_functions(lower.harness_f32(reference_inputs.read("matmul_relu.mlir")))[0]
    p = tileplan.matmul_group_plan(f)
    assert "bias" not in p["buffers"] and p["plan"].off_bias == -1
    tm, tn, tk = p["tile"]
    assert p["buffers"]["init"]["offset"] == 163840 - tm * tn * 4


def _call(plan, A=(64, 32), B=(32, 48), bias=True, act=1):
    lib = npu_amd.lib()
    mA, mB, mo = _mr(list(A)), _mr(list(B)), _mr([A[0], B[1]])
    mb = _mr([B[1]]) if bias else None
    return lib.npu_planned_matmul_bias_act(C.byref(mA), C.byref(mB), C.byref(mb) if mb else None,
                                           C.byref(mo), act, C.byref(plan) if plan else None,
                                           None, None)


def _plan(**kw):
    p = _lib.NpuTilePlan()
    v = dict(tm=32, tn=16, tk=8, lds_bytes=163840, off_a=0, off_a_pong=1024, off_b=2048,
             off_b_pong=2560, off_bias=3072, off_c=4096, off_y=6144)
    v.update(kw)
    for k, x in v.items():
        setattr(p, k, x)
    return p


def test_planned_entry_checks_the_plan_before_launch():
    assert _call(None) == 1 and "plan" in _err()
    assert _call(_plan(tm=160, tn=112)) == 2 and "64 16x16" in _err()
    assert _call(_plan(lds_bytes=200000)) == 1 and "163840" in _err()
    assert _call(_plan(off_y=163840 - 1024)) == 1 and "inside" in _err()
    assert _call(_plan(off_b_pong=1536)) == 1 and "overlap" in _err()
    assert _call(_plan(off_c=4098)) == 1 and "aligned" in _err()
    assert _call(_plan(off_bias=-1)) == 1 and "bias" in _err()
    assert _call(_plan(), bias=False) == 1 and "bias" in _err()
    assert _call(_plan(), A=(64, 30), B=(31, 48)) == 1 and "expected K" in _err()


def test_plan_that_spills_is_refused():
    """At an SRAM size the group's slices do not fit, the reference's
    allocator spills a buffer to DRAM; a launch has no DRAM buffers to place,
    so the plan is refused by name instead of launched."""
    f = mlir.parse_functions(blocks.matmul_bias_act(256, 512, 256, act="relu"))[0]
    with pytest.raises(NotImplementedError, match="spills"):
        tileplan.matmul_group_plan(f, sram=16384)
