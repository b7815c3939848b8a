"""The restated cost model (libnpu_host.so) against known answers.

The known answers are the reference's formulas (lib/Analysis/CostModel.cpp)
evaluated by hand at the reference's default target on the reference's own
test inputs (test/ and test/lit/, read in place by tests/reference_inputs.py):
* roofline of test/lit/cost_evaluate.mlir (CostModel.cpp:174-226): the walk
  counts linalg.fill as 1024 MACs, so 33 556 480 FLOP over 589 824 bytes,
  AI 56.89, 1.8432e-5 s, memory-bound against the ridge of 128;
* best tile configs (CostModel.cpp:346-438) for the matmul of
  test/matmul_relu.mlir, the matmul+bias+ReLU configuration in f32 and the
  conv of test/conv2d_relu.mlir, and the ReLU generics;
* the three-engine subgraph model (CostModel.cpp:829-951) for {matmul, relu}.
Each number is also recomputed here from the formula's terms, so a wrong
term in the C++ shows up as a mismatch in a named quantity.
"""

import pytest

import reference_inputs
from npu_amd import host, mlir



def load(name):
    return host.Graph(mlir.parse_file(reference_inputs.path(name))[0])


@pytest.fixture(scope="module")
def npu():
    return host.default_target()


def test_default_target_is_the_reference_npu(npu):
    d = npu.as_dict()
    assert d["num_cores"] == 6 and d["sram_per_core"] == 2 * 1024 * 1024
    assert d["dram_bandwidth"] == 32 and d["matrix_throughput"] == 4096
    assert d["dsp_throughput"] == 256 and d["clock_ghz"] == 1.0


def test_tile_candidates():
    assert host.tile_candidates(128) == [128, 64, 32, 16]
    assert host.tile_candidates(56) == [56, 28, 16]
    assert host.tile_candidates(24) == [24, 16]
    assert host.tile_candidates(1) == [1]
    assert host.tile_candidates(512) == [512, 256, 128, 64, 32, 16]


def test_roofline_cost_evaluate_kat(npu):
    g = load("lit/cost_evaluate.mlir")
    cm = host.CostModel(g, npu)
    fill, mm = g.find("linalg.fill"), g.find("linalg.matmul")
    assert cm.op_macs(mm) == 128 * 512 * 256
    assert cm.op_macs(fill) == 1024  # not a matmul/conv/generic: the default
    r = cm.roofline([fill, mm])
    assert r.flops == 33_554_432 + 2_048
    # external: init (empty) + A + B in, matmul result out; fill result internal
    assert r.mem_bytes == 128 * 512 * 2 + 128 * 256 * 2 + 256 * 512 * 2 + 128 * 512 * 2 == 589_824
    assert r.arithmetic_intensity == 33_556_480 / 589_824 and round(r.arithmetic_intensity, 2) == 56.89
    assert abs(r.time_sec - 589_824 / 32e9) < 1e-12 and abs(r.time_sec - 1.8432e-5) < 1e-12
    assert r.is_memory_bound  # ridge 4096e9 / 32e9 = 128


def test_best_tile_matmul_kat(npu):
    g = load("matmul_relu.mlir")  # 128x256 . 256x512, f16
    cm = host.CostModel(g, npu)
    best = cm.best_tile_config(g.find("linalg.matmul"))
    assert best.tiles == [128, 256, 16]
    assert best.num_tiles == 1 * 2 * 16 == 32
    a, b, c = 128 * 16 * 2, 16 * 256 * 2, 128 * 256 * 2
    assert best.sram_peak_bytes == 2 * a + 2 * b + c == 90_112
    din, comp, dout = (a + b) // 32, 128 * 256 * 16 // 4096, c // 32
    assert best.total_cycles == din + 31 * max(din, comp) + comp + dout == 14_464


def test_best_tile_matmul_f32_config_kat(npu):
    t = mlir.parse_functions("""
func.func @c1(%A: tensor<256x512xf32>, %B: tensor<512x256xf32>) -> tensor<256x256xf32> {
  %cst = arith.constant 0.0 : f32
  %init = tensor.empty() : tensor<256x256xf32>
  %fill = linalg.fill ins(%cst : f32) outs(%init : tensor<256x256xf32>) -> tensor<256x256xf32>
  %mm = linalg.matmul ins(%A, %B : tensor<256x512xf32>, tensor<512x256xf32>)
                      outs(%fill : tensor<256x256xf32>) -> tensor<256x256xf32>
  return %mm : tensor<256x256xf32>
}""")[0]
    g = host.Graph(t)
    best = host.CostModel(g, npu).best_tile_config(g.find("linalg.matmul"))
    assert best.tiles == [256, 256, 16]
    assert (best.total_cycles, best.num_tiles, best.sram_peak_bytes) == (41_216, 32, 327_680)


def test_best_tile_conv_kat(npu):
    g = load("conv2d_relu.mlir")
    best = host.CostModel(g, npu).best_tile_config(g.find("linalg.conv_2d_nchw_fchw"))
    assert best.tiles == [1, 64, 28, 28]
    inp, w, out = 1 * 64 * 30 * 30 * 2, 64 * 64 * 9 * 2, 64 * 28 * 28 * 2
    assert best.sram_peak_bytes == 2 * inp + w + out == 404_480
    din, comp, dout = (inp + w) // 32, 64 * 28 * 28 * 64 * 9 // 4096, out // 32
    assert best.num_tiles == 4
    assert best.total_cycles == din + 3 * max(din, comp) + comp + dout == 37_264


def test_best_tile_generic_kat(npu):
    g = load("matmul_relu.mlir")  # relu over 128x512 f16
    best = host.CostModel(g, npu).best_tile_config(g.find("linalg.generic"))
    assert best.tiles == [16] and best.num_tiles == 8 and best.total_cycles == 13_856
    t = mlir.parse_functions("""
func.func @r(%x: tensor<256x256xf32>) -> tensor<256x256xf32> {
  %e = tensor.empty() : tensor<256x256xf32>
  %r = linalg.generic {indexing_maps = [affine_map<(d0, d1) -> (d0, d1)>, affine_map<(d0, d1) -> (d0, d1)>],
    iterator_types = ["parallel", "parallel"]} ins(%x : tensor<256x256xf32>) outs(%e : tensor<256x256xf32>) {
  ^bb0(%in: f32, %out: f32):
    %z = arith.constant 0.0 : f32
    %m = arith.maximumf %in, %z : f32
    linalg.yield %m : f32
  } -> tensor<256x256xf32>
  return %r : tensor<256x256xf32>
}""")[0]
    g2 = host.Graph(t)
    best2 = host.CostModel(g2, npu).best_tile_config(g2.find("linalg.generic"))
    row = 256 * 4 * 3
    dma = 16 * row // 32
    assert best2.tiles == [16] and best2.num_tiles == 16
    assert best2.total_cycles == dma + 15 * dma + 16 + dma == 26_128


def test_subgraph_matmul_relu_kat(npu):
    g = load("matmul_relu.mlir")
    cm = host.CostModel(g, npu)
    mm, relu = g.find("linalg.matmul"), g.find("linalg.generic")
    s = cm.subgraph([mm, relu])
    assert (s.matrix_cycles, s.dsp_cycles) == (4096, 256)
    assert s.dma_in_cycles == (65536 + 262144 + 131072 + 131072) // 32 == 18_432
    assert s.dma_out_cycles == 4096
    assert (s.pipelined_cycles, s.unpipelined_cycles) == (22_528, 26_880)
    assert cm.subgraph([mm]).pipelined_cycles == 18_432
    assert cm.subgraph([relu]).pipelined_cycles == 12_288
    assert cm.subgraph_fusion_profitable([mm, relu]) == (True, 8_192)


def test_fusion_profitable_never_into_matrix_consumer(npu):
    g = load("mlp.mlir")
    cm = host.CostModel(g, npu)
    relu1, mm2 = g.find("linalg.generic", 0), g.find("linalg.matmul", 1)
    assert cm.fusion_profitable(relu1, mm2) == (False, 0)
    mm1 = g.find("linalg.matmul", 0)
    fuse, benefit = cm.fusion_profitable(mm1, relu1)
    # benefit = the DRAM round trip of the 128x512 f16 intermediate
    assert fuse and benefit == 2 * (128 * 512 * 2 // 32)


def test_tile_alignment(npu):
    g = load("matmul_relu.mlir")
    cm = host.CostModel(g, npu)
    assert cm.tile_alignment([g.find("linalg.matmul"), g.find("linalg.generic")]) == (True, 0)


def test_spill_strategy(npu):
    # spill costs 2 DMA passes of the intermediate, retile one pass of the tile
    assert host.spill_strategy(npu, 64 * 1024, 16 * 1024) == "spill"
    assert host.spill_strategy(npu, 16 * 1024, 16 * 1024) == "retile"


def test_specs_match_reference_tables(npu):
    g = load("conv2d_relu.mlir")
    cm = host.CostModel(g, npu)
    conv = g.find("linalg.conv_2d_nchw_fchw")
    assert cm.spec_splits(conv) == [(0, 0, True), (1, 1, True), (2, 2, True), (3, 3, True),
                                    (-1, 4, False)]
    mm = host.Graph(mlir.parse_file(reference_inputs.path("matmul_relu.mlir"))[0])
    cmm = host.CostModel(mm, npu)
    assert cmm.spec_splits(mm.find("linalg.matmul")) == [(0, 0, True), (1, 1, True),
                                                         (-1, 2, False)]
    assert cmm.spec_splits(mm.find("linalg.generic")) == [(0, 0, True), (1, 1, True)]


def test_spatial_split_detailed_shared_and_halo(npu):
    g = load("lit/spatial_tiling_conv2d.mlir")
    cm = host.CostModel(g, npu)
    conv = g.find("linalg.conv_2d_nchw_fchw")
    host.spec_reset()  # this 3x3 conv is the first asked about: its spec is in force
    co = cm.spatial_split_detailed(conv, 1, 6)   # split Co: input shared, filter split
    assert co.shared_data_bytes == 1 * 64 * 58 * 58 * 2
    assert co.split_data_bytes == 64 * 64 * 9 * 2 * 11 // 64
    ho = cm.spatial_split_detailed(conv, 2, 6)   # split Ho: input with a 2-row halo
    assert ho.halo_overhead_bytes == 1 * 64 * 58 * 58 * 2 * 2 // 58
    red = cm.spatial_split_detailed(conv, 4, 6)  # split Ci: reduction
    assert red.needs_reduce


def test_mi355x_target():
    t = host.mi355x_target(16).as_dict()
    assert t["num_cores"] == 256 and t["sram_per_core"] == 160 * 1024
    assert t["clock_ghz"] == 2.4 and t["matrix_throughput"] == 2048
    assert host.mi355x_target(32).matrix_throughput == 128
    assert host.mi355x_target(8).matrix_throughput == 4096
    # per-CU rates times 256 CUs x 2.4 GHz x 2 FLOP/MAC give the published peaks
    for bits, peak in ((32, 157.3e12), (16, 2.5166e15), (8, 5.033e15)):
        mac = host.mi355x_target(bits).matrix_throughput
        assert abs(2 * mac * 256 * 2.4e9 / peak - 1) < 0.002


def test_bad_ids_raise():
    g = load("matmul_relu.mlir")
    cm = host.CostModel(g, host.default_target())
    cm.g.op_id.append(999)
    with pytest.raises(ValueError):
        cm.op_macs(len(cm.g.op_id) - 1)


# ---- MI355X launch model (npu_cm_predict_launch) -------------------------
def _plan(**kw):
    from npu_amd._lib import NpuLaunchPlan
    p = NpuLaunchPlan()
    p.kernel = b"test"
    p.grid, p.wg_per_cu, p.tiles, p.load_phases, p.mfma_bits = 256, 1, 256, 0, 16
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_launch_model_hbm_bound():
    """A plan whose only cost is HBM bytes takes bytes / copy bandwidth."""
    g = host.mi355x_gpu()
    c = host.predict_launch(_plan(hbm_bytes=4.3e9), g)
    assert host.BOUNDS[c.bound] == "hbm"
    assert c.time_us == pytest.approx(4.3e9 / (g.hbm_gbs * 1e3))


def test_launch_model_measured_constants():
    """The MI355X constants are npu_calibrate's measurements (sustained clock
    under MFMA load, vector issue rates, LDS/L2/burst rates, latency)."""
    g = host.mi355x_gpu()
    assert (g.cus, g.clock_ghz, g.valu_instr_per_clk_cu, g.wave_valu_clk) == (256, 2.37, 2.0, 8.0)
    assert (g.lds_bytes_per_clk_cu, g.l2_bytes_per_clk_cu, g.burst_bytes_per_clk_cu) == (204.0, 51.0, 34.4)
    assert list(g.mfma_macs_per_clk_cu) == [128.0, 2048.0, 4096.0]


def test_launch_model_compute_streams():
    """MFMA and vector-ALU issue add up on a SIMD; LDS is the other stream.
    A tile's vector instructions are spread over the four SIMDs; one wave
    issues one every 8 clocks, a SIMD with four or more waves one every 2."""
    g = host.mi355x_gpu()
    clk = g.clock_ghz * 1e3
    # 2048*1000 bf16 MACs = 1000 clocks of MFMA; 500 instructions = 125 per SIMD
    one = host.predict_launch(_plan(tile_macs=2048.0 * 1000, tile_valu=500.0), g)
    assert one.tile_compute_us == pytest.approx((1000 + 125 * 8) / clk)          # one wave per SIMD
    four = host.predict_launch(_plan(tile_macs=2048.0 * 1000, tile_valu=500.0, wg_per_cu=4,
                                     grid=1024, tiles=1024), g)
    assert four.tile_compute_us == pytest.approx((1000 + 125 * 2) / clk)         # four waves per SIMD
    assert host.BOUNDS[four.bound] == "mfma"
    # LDS-bound: 4000 clocks of LDS reads
    c = host.predict_launch(_plan(tile_macs=2048.0 * 10, tile_lds_bytes=g.lds_bytes_per_clk_cu * 4000,
                                  wg_per_cu=2, grid=512, tiles=512), g)
    assert c.tile_compute_us == pytest.approx(4000 / clk) and host.BOUNDS[c.bound] == "lds"
    # f32 is 16x slower per MAC than bf16
    c32 = host.predict_launch(_plan(tile_macs=128.0 * 1000, mfma_bits=32), g)
    assert c32.tile_compute_us == pytest.approx(1000 / clk)


def test_launch_model_rounds_and_occupancy():
    """n tiles per CU: a workgroup runs its tiles one after another (its
    waves' streams in order, after its load), so k resident workgroups take
    ceil(n / k) rounds of that serial time, unless the CU's MFMA stream binds
    first."""
    g = host.mi355x_gpu()
    clk = g.clock_ghz * 1e3
    lat = g.mem_latency_us * clk
    base = dict(tiles=256 * 8, tile_macs=2048.0 * 3000, load_phases=1)
    one = host.predict_launch(_plan(wg_per_cu=1, grid=256, **base), g)
    two = host.predict_launch(_plan(wg_per_cu=2, grid=512, **base), g)
    serial = lat + 3000
    assert one.tiles_per_cu == 8 and one.tile_serial_us == pytest.approx(serial / clk)
    assert one.cu_us == pytest.approx(8 * serial / clk)                       # 8 rounds
    assert host.BOUNDS[one.bound] == "latency"
    # two workgroups: 4 rounds of serial time, against 8 x 3000 clocks of MFMA
    assert two.cu_us == pytest.approx(max(4 * serial, 8 * 3000) / clk)
    # ragged: 3 tiles on a CU with 2 workgroups take 2 rounds
    rag = host.predict_launch(_plan(wg_per_cu=2, grid=512, tiles=256 * 3, load_phases=1,
                                    tile_macs=2048.0 * 10), g)
    assert rag.cu_us == pytest.approx(2 * (lat + 10) / clk)


def test_launch_model_setup_burst():
    """Setup data (filters fetched once per workgroup) costs a latency plus
    the k resident workgroups' bytes at the all-CU burst rate; none without."""
    g = host.mi355x_gpu()
    clk = g.clock_ghz * 1e3
    base = dict(tiles=256, tile_macs=2048.0 * 10, wg_per_cu=2, grid=512)
    none = host.predict_launch(_plan(**base), g)
    some = host.predict_launch(_plan(wg_setup_bytes=34.4 * 1000, **base), g)
    assert some.cu_us - none.cu_us == pytest.approx(g.mem_latency_us + 2 * 1000 / clk)


def test_launch_model_rejects_empty_plan():
    with pytest.raises(ValueError):
        host.predict_launch(_plan(grid=0))


def test_block_prediction_adds_launch_cost():
    g = host.mi355x_gpu()
    plans = [_plan(hbm_bytes=1e6), _plan(hbm_bytes=2e6)]
    total, parts = host.predict_block(plans, g)
    assert total == pytest.approx(sum(c.time_us for _, c in parts) + 2 * g.launch_us)
