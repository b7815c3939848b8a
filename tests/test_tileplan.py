"""The reference's memory plan as a launch's LDS layout (CPU side):
npu-barrier-alloc's subgraphs and barrier ids (DMASchedulingPass.cpp:92-147),
the tile loop's buffers of the fill -> matmul -> generic and fill ->
conv_2d_nchw_fchw -> generic groups planned at one CU's LDS (163 840 bytes)
by the dual-end allocator (spills and prefetch regions included), and the
checks the plan-driven entry points make before any launch."""
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


# ---------------------------------------------------------------- the conv group
def _conv_plan(shape, bias=True):
    N, C, F, H, W = shape
    text = (blocks.nchw_conv_bias_act(N, C, F, H, W) if bias
            else lower.harness_f32(blocks.nchw_conv_relu(N, C, F, H, W)))
    return tileplan.conv_group_plan(mlir.parse_functions(text)[0])


def _no_overlap(buffers, sram=163840):
    spans = []
    for v in buffers.values():
        for off in (v["offset"], v["offset_pong"], v["prefetch_addr"]):
            if off >= 0:
                assert off % 4 == 0 and off + v["bytes"] <= sram
                spans.append((off, off + v["bytes"]))
    spans.sort()
    assert all(e <= s for (_, e), (s, _) in zip(spans, spans[1:])), spans


def test_conv_group_plan_conv2d_relu():
    """test/conv2d_relu.mlir's group (the builder's text of it) at the
    reference's default target, one output row per core, SRAM 163 840 bytes.
    The temporal tile of a row is 32 of the 64 output channels (2 tiles).
    By the allocator's rules: the input rows [64][3][58] (44 544 bytes) in
    a ping/pong pair from the low end; the filter slice [32][64][3][3]
    (73 728 bytes) no longer fits beside the two output rows (7 168 bytes
    each, from the high end in first-use order: the accumulator, then the
    output) and is spilled; the prefetch copy of the input rows takes the
    top of the free gap, right below the output row."""
    f = mlir.parse_functions(lower.harness_f32(blocks.reference_workload("conv2d_relu.mlir")))[0]
    p = tileplan.conv_group_plan(f)
    assert p["tile"][:4] == [1, 32, 1, 56] and p["tco"] == 32 and p["tiles"] == 2
    assert p["cores"] == 56
    b = p["buffers"]
    rows, filt, out_row = 64 * 3 * 58 * 4, 32 * 64 * 9 * 4, 32 * 56 * 4
    assert (b["x"]["bytes"], b["w"]["bytes"], b["y"]["bytes"]) == (rows, filt, out_row)
    assert (b["x"]["offset"], b["x"]["offset_pong"]) == (0, rows)
    assert 2 * rows + filt + 2 * out_row > 163840 and b["w"]["spilled"]
    assert (b["w"]["offset"], b["w"]["offset_pong"], b["w"]["prefetch_addr"]) == (-1, -1, -1)
    assert b["init"]["offset"] == 163840 - out_row and b["y"]["offset"] == 163840 - 2 * out_row
    assert b["x"]["prefetch_addr"] == b["y"]["offset"] - rows
    assert "bias" not in b
    _no_overlap(b)
    plan = p["plan"]
    assert (plan.tco, plan.lds_bytes) == (32, 163840)
    assert (plan.off_in, plan.off_in_pong, plan.off_in_prefetch) == (0, rows, b["x"]["prefetch_addr"])
    assert (plan.off_w, plan.off_w_pong, plan.off_w_prefetch) == (-1, -1, -1)
    assert (plan.off_bias, plan.off_bias_pong, plan.off_bias_prefetch) == (-1, -1, -1)
    assert (plan.off_c, plan.off_y) == (b["init"]["offset"], b["y"]["offset"])


@pytest.mark.parametrize("shape", [(2, 5, 45, 64, 19), (2, 24, 36, 50, 27), (1, 64, 96, 112, 20),
                                   (1, 8, 20, 40, 16)])
def test_conv_group_plans_with_bias(shape):
    """Groups with a bias generic (along the output channels): the bias
    slice is a third input of the loop, in its own ping/pong pair; every
    buffer in SRAM is aligned, inside it and apart from the others; a row
    the temporal pass leaves whole (tile count 1) is one tile of all F
    channels."""
    p = _conv_plan(shape)
    N, C, F, H, W = shape
    b = p["buffers"]
    assert b["bias"]["bytes"] == 4 * p["tco"] and b["bias"]["double_buffered"]
    assert p["tiles"] == -(-F // p["tco"]) and p["cores"] == N * H
    _no_overlap(b)
    plan = p["plan"]
    assert (plan.off_bias, plan.off_bias_pong, plan.off_bias_prefetch) == (
        b["bias"]["offset"], b["bias"]["offset_pong"], b["bias"]["prefetch_addr"])
    if shape == (1, 8, 20, 40, 16):
        assert p["tco"] == F and p["tiles"] == 1
    if shape == (1, 64, 96, 112, 20):
        # the filter slice found room for its ping only
        assert b["w"]["offset"] >= 0 and b["w"]["offset_pong"] == -1
        assert plan.off_w_pong == -1


def test_conv_group_plan_refusals():
    """A spatial split the launch does not run (over output channels) and
    a strided conv are refused by name."""
    with pytest.raises(NotImplementedError, match="spatial split"):
        _conv_plan((1, 16, 20, 14, 14))
    f = mlir.parse_functions(blocks.matmul_bias_act(64, 32, 48))[0]
    with pytest.raises(NotImplementedError, match="conv_2d_nchw_fchw"):
        tileplan.conv_group_plan(f)


def _conv_call(plan, x=(1, 4, 10, 12), w=(8, 4, 3, 3), bias=True, act=1, out=None):
    lib = npu_amd.lib()
    out = out or [x[0], w[0], x[2] - w[2] + 1, x[3] - w[3] + 1]
    mx, mw, mo = _mr(list(x)), _mr(list(w)), _mr(out)
    mb = _mr([w[0]]) if bias else None
    return lib.npu_planned_conv2d_nchw_bias_act(C.byref(mx), C.byref(mw),
                                                C.byref(mb) if mb else None, C.byref(mo), act,
                                                C.byref(plan) if plan else None, None, None)


def _cplan(**kw):
    p = _lib.NpuConvTilePlan()
    v = dict(tco=4, lds_bytes=163840, off_in=0, off_in_pong=1024, off_in_prefetch=2048,
             off_w=4096, off_w_pong=5120, off_w_prefetch=6144, off_bias=8192, off_bias_pong=8256,
             off_bias_prefetch=8320, off_c=10240, off_y=11264)
    v.update(kw)
    for k, x in v.items():
        setattr(p, k, x)
    return p


def test_planned_conv_entry_checks_the_plan_before_launch():
    # rows [4][3][12] = 576 bytes, filters [4][4][3][3] = 576, bias 16,
    # C and Y rows [4][10] = 160
    assert _conv_call(None) == 1 and "plan" in _err()
    assert _conv_call(_cplan(tco=0)) == 1 and "tco" in _err()
    assert _conv_call(_cplan(tco=9)) == 1 and "tco" in _err()
    assert _conv_call(_cplan(lds_bytes=200000)) == 1 and "163840" in _err()
    assert _conv_call(_cplan(off_y=163840 - 100)) == 1 and "inside" in _err()
    assert _conv_call(_cplan(off_w_pong=4100)) == 1 and "overlap" in _err()
    assert _conv_call(_cplan(off_bias_prefetch=8192 + 8)) == 1 and "overlap" in _err()
    assert _conv_call(_cplan(off_c=10242)) == 1 and "aligned" in _err()
    assert _conv_call(_cplan(off_c=-1)) == 1 and "C and Y" in _err()
    assert _conv_call(_cplan(off_w=-1)) == 1 and "outside SRAM" in _err()
    assert _conv_call(_cplan(off_bias=-1), bias=False) == 1 and "outside SRAM" in _err()
    assert _conv_call(_cplan(off_bias=-1, off_bias_pong=-1, off_bias_prefetch=-1)) == 1 \
        and "bias" in _err()
    assert _conv_call(_cplan(), bias=False) == 1 and "bias" in _err()
    assert _conv_call(_cplan(), w=(8, 5, 3, 3)) == 1 and "expected C" in _err()
    assert _conv_call(_cplan(), out=[1, 8, 8, 9]) == 1 and "out" in _err()
    assert _conv_call(_cplan(), w=(8, 4, 11, 3), out=[1, 8, 1, 10]) == 1 and "larger" in _err()
    assert _conv_call(_cplan(), act=9) == 1 and "act" in _err()
