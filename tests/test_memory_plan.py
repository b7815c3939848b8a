"""Buffers after tiling (libnpu_host.so): npu-bufferize's DMA insertion,
npu-sram-allocation's dual-end plan, npu-cost-evaluate's record, and the
decision pipeline in the reference's order.

Allocator cases are worked by hand from SRAMAllocationPass.cpp:127-342;
the bufferize contract is test/lit/bufferize_dma.mlir; the SRAM bound is
the reference simulator's check (tools/harness/sram_simulator.py:243-256);
the cost record's roofline numbers are the test/lit/cost_evaluate.mlir KAT.
"""
import json

import pytest

import reference_inputs
from npu_amd import host, mlir, pipeline

IN, OUT, MID = 0, 1, 2


def bufs(*specs):
    """(role, bytes, first_use, last_use, in_loop) tuples -> SramBuffer list."""
    out = []
    for role, nbytes, first, last, loop in specs:
        b = host.SramBuffer()
        b.value, b.role, b.bytes, b.first_use, b.last_use, b.in_loop = -1, role, nbytes, first, last, loop
        out.append(b)
    return out


def test_dual_end_layout_pingpong_and_prefetch():
    # A, B inputs in a tile loop (ping/pong, low end); C output (high end);
    # I intermediate (after the inputs); then the space left prefetches the
    # inputs, largest first, from the high end.
    b = bufs((IN, 100, 0, 10, 1), (IN, 64, 1, 10, 1), (OUT, 10, 2, 10, 1), (MID, 200, 3, 10, 1))
    s = host.sram_allocation(b, 1024)
    A, B, Cc, I = b
    assert (A.addr, A.addr_pong, A.double_buffered) == (0, 128, 1)
    assert (B.addr, B.addr_pong, B.double_buffered) == (256, 320, 1)
    assert Cc.addr == 1024 - 64 and Cc.addr_pong == -1
    assert I.addr == 384
    assert (A.prefetch_addr, B.prefetch_addr) == (960 - 128, 960 - 128 - 64)
    assert (s.spilled, s.prefetched, s.prefetch_bytes, s.free_after) == (0, 2, 192, 320)


def test_dead_buffers_are_reused_and_outputs_kept():
    b = bufs((MID, 512, 0, 1, 1), (MID, 512, 2, 3, 1))
    host.sram_allocation(b, 1024)
    assert b[0].addr == 0 and b[1].addr == 0            # X dead before Y: its space again
    b = bufs((OUT, 256, 0, 1, 1), (MID, 256, 2, 3, 1), (MID, 512, 4, 5, 1))
    host.sram_allocation(b, 1024)
    assert b[0].addr == 768                              # outputs are never released
    assert b[1].addr == 0 and b[2].addr == 0


def test_release_is_from_the_top_of_the_low_end():
    """The reference releases a dead buffer by lowering the low-water mark by
    its size, wherever it sits (DualEndAllocator::freeLow): a later buffer can
    then land on a live one.  Restated as written."""
    b = bufs((IN, 128, 0, 1, 0), (MID, 128, 1, 5, 1), (MID, 128, 2, 5, 1))
    host.sram_allocation(b, 4096)
    assert b[0].addr == 0 and b[1].addr == 128
    assert b[2].addr == 128  # A's release lowered the mark below the live B


def test_spill_and_single_buffer_fallback():
    b = bufs((IN, 2000, 0, 1, 1))
    s = host.sram_allocation(b, 1024)
    assert b[0].spilled and b[0].addr == -1 and s.spilled == 1
    b = bufs((IN, 600, 0, 1, 1))                         # fits once, not twice
    host.sram_allocation(b, 1024)
    assert b[0].addr == 0 and not b[0].double_buffered and b[0].addr_pong == -1


def test_bufferize_inserts_dma_for_loop_operands():
    """test/lit/bufferize_dma.mlir: npu.alloc_sram and a dram_to_sram
    npu.dma_copy for the operands used inside the tile loop."""
    g = host.Graph(mlir.parse_file(reference_inputs.path("lit/bufferize_dma.mlir"))[0])
    b = host.bufferize(g, g.linalg_ops())
    names = {v: k for k, v in g.value_id.items()}
    got = {names[x.value]: (host.ROLES[x.role], x.bytes) for x in b}
    assert got == {"%init": ("output", 128 * 64 * 2), "%A": ("input", 128 * 256 * 2),
                   "%B": ("input", 256 * 64 * 2)}
    assert all(x.in_loop for x in b)
    assert [names[x.value] for x in b] == ["%init", "%A", "%B"]  # first-use order
    # tile-slice sizes replace the full tensors when given
    b2 = host.bufferize(g, g.linalg_ops(), {"%A": 22 * 256 * 2})
    assert [x.bytes for x in b2 if names[x.value] == "%A"] == [22 * 256 * 2]


@pytest.mark.parametrize("path", reference_inputs.all_inputs())
def test_pipeline_plans_fit_the_sram(path):
    """Every reference test input through the pipeline: each planned buffer
    lies inside the SRAM (the simulator's offset + size <= SRAM check), and
    every function emits one COST_JSON line with the reference's keys."""
    keys = ["name", "flops", "mem_bytes", "arithmetic_intensity", "time_sec", "is_memory_bound",
            "efficiency", "dma_in_bytes", "dma_out_bytes", "matrix_cycles", "dsp_cycles",
            "peak_sram_bytes", "num_tile_iterations", "num_linalg_ops", "sram_budget", "bottleneck"]
    t = host.default_target()
    for rep in pipeline.run_file(reference_inputs.path(path), t):
        assert rep["steps"][0] == "fusion" and rep["steps"][-1] == "cost-eval"
        assert len(rep["cost_json"]) == len(rep["functions"])
        for f, line in zip(rep["functions"], rep["cost_json"]):
            assert line.startswith("COST_JSON: ")
            rec = json.loads(line[len("COST_JSON: "):])
            assert list(rec) == keys and rec["name"] == f["name"]
            for b in f["sram"]["buffers"]:
                if not b["spilled"]:
                    assert 0 <= b["offset"] and b["offset"] + b["bytes"] <= t.sram_per_core
                    if b["double_buffered"]:
                        assert b["offset_pong"] + b["bytes"] <= t.sram_per_core


def test_cost_record_roofline_kat():
    """test/lit/cost_evaluate.mlir: the walk also counts linalg.fill at the
    default 1024 MACs: 33 554 432 + 2 048 FLOP over 589 824 bytes."""
    rep = pipeline.run_file(reference_inputs.path("lit/cost_evaluate.mlir"))[0]
    rec = json.loads(rep["cost_json"][0][len("COST_JSON: "):])
    assert rec["flops"] == 33556480 and rec["mem_bytes"] == 589824
    assert rec["arithmetic_intensity"] == pytest.approx(33556480 / 589824)
    assert rec["time_sec"] == pytest.approx(1.8432e-5) and rec["bottleneck"] == "memory"
    assert rec["num_linalg_ops"] == 2 and rec["sram_budget"] == 2 * 1024 * 1024


def test_pipeline_maps_groups_to_entry_points():
    rep = pipeline.run_file(reference_inputs.path("matmul_relu.mlir"))[0]
    (f,) = rep["functions"]
    assert f["name"] == "fused_fill_matmul_generic_0"
    assert f["entry_point"] == "fused_matmul_bias_act"
    assert f["temporal"][0]["tiles"] == [128, 256, 16]   # the best-tile KAT


def disjoint(b):
    """No two buffers live at the same time share a byte (ping and pong included)."""
    spans = []
    for x in b:
        if x.spilled:
            continue
        for a in (x.addr, x.addr_pong):
            if a >= 0:
                spans.append((a, a + x.bytes, x.first_use, x.last_use))
    for i, (a0, a1, f0, l0) in enumerate(spans):
        for b0, b1, f1, l1 in spans[i + 1:]:
            if f0 <= l1 and f1 <= l0:
                assert a1 <= b0 or b1 <= a0, (a0, a1, b0, b1)


# The workgroup LDS buffers of the MI355X kernels, written as one tile loop's
# buffers (role, bytes, first use, last use, ping/pong in the loop) and planned
# by the dual-end allocator at one CU's 160 KiB.  The plan's footprint (low end
# plus high end), rounded up to the 512-byte LDS allocation granule, is the
# LDS size the kernel trace reports for the compiled kernel.  The kernels hold
# the next tile's prefetch in registers, so the prefetch copies the allocator
# places in the space left are not part of the footprint.
LDS_KERNELS = {
    # xs[100 x 36 floats], wds[9 x 144], es[100 x 152]
    "irb_kernel<24, 144>": ([(IN, 100 * 36 * 4, 0, 9, 0), (IN, 9 * 144 * 4, 1, 9, 0),
                             (MID, 100 * 152 * 4, 2, 5, 0)], 80384),
    # halo[4 rows x 58 px x 160 B] plus a 16-byte trash slot per lane,
    # ostage[2 x 56 px x 160 B]
    "conv3x3_stream_kernel bf16 C=64": ([(IN, 4 * 58 * 160 + 64 * 16, 0, 5, 0),
                                         (OUT, 2 * 56 * 160, 1, 6, 0)], 56320),
    # f32 on the bf16 pipe: a ring of 6 halo row slots [58 px x 416 B] plus
    # 8-byte trash slots (768 B), and the partial-sum exchange [4 filter
    # groups x 4 blocks x 1 KiB] (the filters' staging before the walk)
    "conv3x3_x6_kernel<56, 2, 56>": ([(IN, 6 * 58 * 416 + 768, 0, 9, 0),
                                      (MID, 4 * 4 * 1024, 1, 9, 0)], 162304),
    # xs[112 x 288 B], y1[112 x 96 B], y2[64 x 96 B]
    "qbottleneck_kernel<256, 64>": ([(IN, 112 * 288, 0, 9, 0), (MID, 112 * 96, 1, 4, 0),
                                     (MID, 64 * 96, 2, 6, 0)], 49152),
    # A[64 x 144 bf16] and B[64 x 144 bf16] ping/pong, inv_rms[64 floats]
    # (64-row tiles of eight waves)
    "llama_gemm_kernel<1, 0, 8> (rmsnorm prologue)": ([(IN, 64 * 144 * 2, 0, 9, 1),
                                                       (IN, 64 * 144 * 2, 1, 9, 1),
                                                       (MID, 64 * 4, 2, 9, 0)], 74240),
    # A[32 x 144 bf16] and B[64 x 144 bf16] ping/pong (32-row tiles, four waves)
    "llama_gemm_kernel<0, 1, 4> (no prologue)": ([(IN, 32 * 144 * 2, 0, 9, 1),
                                                  (IN, 64 * 144 * 2, 1, 9, 1)], 55296),
    # two B operands (gate and up) for the SwiGLU epilogue
    "llama_gemm_kernel<1, 2, 8> (swiglu)": ([(IN, 64 * 144 * 2, 0, 9, 1), (IN, 64 * 144 * 2, 1, 9, 1),
                                             (IN, 64 * 144 * 2, 2, 9, 1),
                                             (MID, 64 * 4, 3, 9, 0)], 111104),
    # the single-panel RMSNorm GEMMs (K <= 512): the normalised A panel
    # [4 chunks x 64 x 144 bf16] and B [64 x 144 bf16] ping/pong (two for SwiGLU)
    "llama_norm_gemm_kernel<0> (qkv, one panel)": ([(IN, 4 * 64 * 144 * 2, 0, 9, 0),
                                                    (IN, 64 * 144 * 2, 1, 9, 1)], 110592),
    "llama_norm_gemm_kernel<2> (swiglu, one panel)": ([(IN, 4 * 64 * 144 * 2, 0, 9, 0),
                                                       (IN, 64 * 144 * 2, 1, 9, 1),
                                                       (IN, 64 * 144 * 2, 2, 9, 1)], 147456),
    # K[4 key groups x 64 x 80 bf16] and V^T[4 x 64 x 80 bf16] ping/pong
    "llama_attention_kernel": ([(IN, 4 * 64 * 80 * 2, 0, 9, 1), (IN, 4 * 64 * 80 * 2, 1, 9, 1)], 163840),
}


@pytest.mark.parametrize("name", sorted(LDS_KERNELS))
def test_lds_plans_of_the_kernels(name):
    specs, traced = LDS_KERNELS[name]
    lds = 160 * 1024
    b = bufs(*specs)
    s = host.sram_allocation(b, lds)
    assert s.spilled == 0
    disjoint(b)
    low = max([x.addr + x.bytes for x in b if x.role != OUT] +
              [x.addr_pong + x.bytes for x in b if x.addr_pong >= 0])
    high = lds - min([x.addr for x in b if x.role == OUT], default=lds)
    assert (low + high + 511) // 512 * 512 == traced


NPU_TARGET_TEXT = """
#big = #npu.target<num_cores = 8, sram_per_core = 163840, dram_bandwidth = 8000,
                   sram_bandwidth = 1024, matrix_throughput = 2048, dsp_throughput = 512,
                   dma_channels = 4>
module attributes {npu.target = #big} {
""" + '''  func.func @mm(%A: tensor<128x256xf32>, %B: tensor<256x512xf32>) -> tensor<128x512xf32> {
    %cst = arith.constant 0.0 : f32
    %init = tensor.empty() : tensor<128x512xf32>
    %fill = linalg.fill ins(%cst : f32) outs(%init : tensor<128x512xf32>) -> tensor<128x512xf32>
    %mm = linalg.matmul ins(%A, %B : tensor<128x256xf32>, tensor<256x512xf32>)
                        outs(%fill : tensor<128x512xf32>) -> tensor<128x512xf32>
    return %mm : tensor<128x512xf32>
  }
}
'''


def test_module_target_attribute_retargets_the_pipeline():
    """#npu.target on the module (NPUDialect.td:100-113) replaces the seven
    parameters of the default target, as CostModelAnalysis does
    (CostModel.cpp:985-1000); the other fields keep their defaults."""
    f = mlir.parse_functions(NPU_TARGET_TEXT)[0]
    assert f.target == {"num_cores": 8, "sram_per_core": 163840, "dram_bandwidth": 8000,
                        "sram_bandwidth": 1024, "matrix_throughput": 2048, "dsp_throughput": 512,
                        "dma_channels": 4}
    rep = pipeline.run(f)
    t = rep["target"]
    assert t["num_cores"] == 8 and t["sram_per_core"] == 163840 and t["dram_bandwidth"] == 8000
    d = host.default_target().as_dict()
    assert t["clock_ghz"] == d["clock_ghz"] and t["noc_bandwidth"] == d["noc_bandwidth"]
    # the SRAM plan and cost record use the module's target
    rec = json.loads(rep["cost_json"][0][len("COST_JSON: "):])
    assert rec["sram_budget"] == 163840
    # the same function without the attribute: the default NPU
    plain = mlir.parse_functions(NPU_TARGET_TEXT[NPU_TARGET_TEXT.index("  func.func"):]
                                 .rsplit("}", 1)[0])[0]
    assert plain.target is None
    assert json.loads(pipeline.run(plain)["cost_json"][0][len("COST_JSON: "):])["sram_budget"] \
        == 2 * 1024 * 1024


def test_inline_target_and_errors():
    txt = NPU_TARGET_TEXT.replace("#big = #npu.target", "#unused = #npu.target").replace(
        "npu.target = #big", "npu.target = #npu.target<num_cores = 2, sram_per_core = 4096, "
        "dram_bandwidth = 1, sram_bandwidth = 2, matrix_throughput = 3, dsp_throughput = 4, "
        "dma_channels = 1>")
    assert mlir.parse_target(txt)["num_cores"] == 2
    with pytest.raises(ValueError, match="missing"):
        mlir.parse_target("module attributes {npu.target = #npu.target<num_cores = 2>} {}")
    with pytest.raises(ValueError, match="does not define"):
        mlir.parse_target("module attributes {npu.target = #nowhere} {}")
