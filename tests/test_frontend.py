"""Frontends (npu_amd.frontend): a torch module traced to NHWC linalg, and the
reference's NCHW model-zoo texts rewritten to NHWC, both run by the host
lowering.  (The GPU runs of these programs are in test_gpu_parity.py.)"""

import pytest
import torch
import torch.nn as nn

import reference_inputs
from npu_amd import blocks, frontend, lower, mlir


class BasicBlock(nn.Module):
    """ResNet basic block (inference): conv3x3-BN-ReLU, conv3x3-BN, + x, ReLU."""

    def __init__(self, C):
        super().__init__()
        self.c1, self.b1 = nn.Conv2d(C, C, 3, padding=1, bias=False), nn.BatchNorm2d(C)
        self.c2, self.b2 = nn.Conv2d(C, C, 3, padding=1, bias=False), nn.BatchNorm2d(C)
        self.relu = nn.ReLU()

    def forward(self, x):
        y = self.relu(self.b1(self.c1(x)))
        return self.relu(self.b2(self.c2(y)) + x)


class InvertedResidual(nn.Module):
    """MobileNetV2 inverted residual block of stride 1, without batch norm."""

    def __init__(self, C, E):
        super().__init__()
        self.expand = nn.Conv2d(C, E, 1, bias=False)
        self.dw = nn.Conv2d(E, E, 3, padding=1, groups=E, bias=False)
        self.project = nn.Conv2d(E, C, 1, bias=False)
        self.act = nn.ReLU6()

    def forward(self, x):
        return self.project(self.act(self.dw(self.act(self.expand(x))))) + x


class MLP(nn.Module):
    def __init__(self, K, H, N):
        super().__init__()
        self.l1, self.l2 = nn.Linear(K, H), nn.Linear(H, N)
        self.relu = nn.ReLU()

    def forward(self, x):
        return self.relu(self.l2(self.relu(self.l1(x))))


def randomize_bn(m, seed=0):
    g = torch.Generator().manual_seed(seed)
    for bn in [x for x in m.modules() if isinstance(x, nn.BatchNorm2d)]:
        bn.running_mean.uniform_(-0.1, 0.1, generator=g)
        bn.running_var.uniform_(0.5, 1.5, generator=g)
        bn.weight.data.uniform_(0.5, 1.5, generator=g)
        bn.bias.data.uniform_(-0.1, 0.1, generator=g)
    return m


def test_torch_basic_block_is_two_conv_calls():
    """Batch norm folds into the convs' filters and biases; the second conv's
    generic holds the bias, the residual and the ReLU."""
    torch.manual_seed(0)
    m = randomize_bn(BasicBlock(64))
    text, params = frontend.from_torch(m, torch.rand(2, 64, 8, 8), name="basic_block")
    prog = lower.lower_text(text)
    assert [(c.entry, c.params) for c in prog.calls] == [
        ("fused_conv2d_nhwc_bias_act", {"pad": 1, "act": "relu"}),
        ("fused_conv2d_nhwc_bias_res_act", {"pad": 1, "act": "relu"})]
    assert prog.calls[1].args[3] == "%x0"
    assert list(params["x0"].shape) == [2, 8, 8, 64] and list(params["w1"].shape) == [64, 3, 3, 64]
    # the folded filter: w * gamma / sqrt(var + eps), channels last
    bn = m.b1
    s = bn.weight / torch.sqrt(bn.running_var + bn.eps)
    want = (m.c1.weight * s.view(-1, 1, 1, 1)).permute(0, 2, 3, 1)
    assert torch.allclose(params["w1"], want, rtol=1e-6, atol=1e-7)


def test_torch_inverted_residual_is_the_fused_irb_call():
    m = InvertedResidual(24, 144)
    text, params = frontend.from_torch(m, torch.rand(1, 24, 9, 13))
    (c,) = lower.lower_text(text).calls
    assert c.entry == "fused_irb_f32" and list(params["w2"].shape) == [3, 3, 144]


def test_torch_mlp_is_a_matmul_chain():
    text, params = frontend.from_torch(MLP(64, 128, 32), torch.rand(16, 64))
    prog = lower.lower_text(text)
    assert prog.entry_points == ["fused_matmul_bias_act", "fused_matmul_bias_act"]
    assert list(params["w1"].shape) == [64, 128]   # nn.Linear's [out, in], transposed


class _ScaledResidual(nn.Module):
    """conv -> torch.add(y, x, alpha=2): the residual is scaled, not added."""

    def __init__(self):
        super().__init__()
        self.c = nn.Conv2d(16, 16, 3, padding=1)

    def forward(self, x):
        return torch.relu(torch.add(self.c(x), x, alpha=2))


def test_torch_add_with_alpha_is_refused():
    with pytest.raises(NotImplementedError, match="alpha"):
        frontend.from_torch(_ScaledResidual(), torch.rand(1, 16, 8, 8))


@pytest.mark.parametrize("module,why", [
    (nn.Sequential(nn.Conv2d(16, 16, 3, stride=2, padding=1)), "stride"),
    (nn.Sequential(nn.Conv2d(16, 16, 3, padding=1, groups=4)), "grouped"),
    (nn.Sequential(nn.Conv2d(16, 16, 3, padding=1), nn.MaxPool2d(2)), "MaxPool2d"),
    (nn.Sequential(nn.Conv2d(16, 16, 3, padding=1), nn.Sigmoid()), "Sigmoid"),
])
def test_torch_frontend_refuses_what_no_entry_point_runs(module, why):
    with pytest.raises(NotImplementedError, match=why):
        frontend.from_torch(module, torch.rand(1, 16, 8, 8))


def _form(fn):
    """Op-by-op form of a function: names, types, maps, iterators, body
    constants, pads and strides (SSA names aside)."""
    out = []
    for op in fn.ops:
        d = (op.name, tuple(str(fn.types[r]) for r in op.results),
             tuple(str(fn.types.get(v)) for v in op.ins + op.outs + op.operands))
        if op.name == "linalg.generic":
            d += (str(op.attrs["maps"]), tuple(op.iterators),
                  tuple((b.name, b.value if b.name == "arith.constant" else None)
                        for b in op.attrs["body"]))
        if op.name == "tensor.pad":
            d += (tuple(op.attrs["low"]), tuple(op.attrs["high"]))
        if "conv" in op.name:
            d += (tuple(op.attrs.get("strides", [1, 1])),)
        out.append(d)
    return out


@pytest.mark.parametrize("model,inp,out,args,ours", [
    ("mobilenetv2.mlir", "%conv28", "%add44",
     ["%conv28", "%w_blk2_exp", "%w_blk2_dw", "%w_blk2_proj"],
     lambda: blocks.model_zoo_irb(1, 24, 144, 56, 56)),
    ("resnet50.mlir", "%relu32", "%relu50",
     ["%relu32", "%w_s0_b1_c1", "%w_s0_b1_c2", "%w_s0_b1_c3"],
     lambda: blocks.model_zoo_bottleneck(1, 256, 64, 56, 56, True)),
])
def test_model_zoo_block_builder_is_the_reference_block(model, inp, out, args, ours):
    """blocks.model_zoo_bottleneck writes the form of the reference's
    model-zoo blocks -- mobilenetv2.mlir's inverted residual block 2
    (:166-226), resnet50.mlir's second stage-0 bottleneck (:194-267) -- op for
    op: the same ops, types, maps, bodies, pads and strides."""
    ref = mlir.parse_functions(reference_inputs.read("models/" + model))[0]
    blk = frontend.extract_block(ref, [inp], out)
    assert [a for a, _ in blk.args] == args
    assert _form(mlir.parse_functions(ours())[0]) == _form(blk)


def test_nchw_to_nhwc_permutes_shapes_maps_and_pads():
    f = mlir.parse_functions(lower.harness_f32(blocks.model_zoo_irb(2, 24, 144, 7, 9)))[0]
    g = frontend.nchw_to_nhwc(f)
    assert [str(t) for _, t in g.args] == ["tensor<2x7x9x24xf32>", "tensor<144x1x1x24xf32>",
                                           "tensor<144x3x3x144xf32>", "tensor<24x1x1x144xf32>"]
    pads = [op for op in g.ops if op.name == "tensor.pad"]
    assert pads[0].attrs["low"] == [0, 1, 1, 0] and pads[0].attrs["high"] == [0, 1, 1, 0]
    assert all(op.name != "linalg.conv_2d_nchw_fchw" for op in g.ops)
    # a channel bias: map (d1) over NCHW becomes (d3) over NHWC
    text = frontend.emit(g)
    assert mlir.parse_functions(text)[0].ops[0].name == g.ops[0].name
    bias_text = ("func.func @b(%x: tensor<1x8x4x5xf32>, %b: tensor<8xf32>) -> tensor<1x8x4x5xf32> {\n"
                 "  %e = tensor.empty() : tensor<1x8x4x5xf32>\n"
                 "  %y = linalg.generic {indexing_maps = [affine_map<(d0, d1, d2, d3) -> (d0, d1, d2, d3)>, "
                 "affine_map<(d0, d1, d2, d3) -> (d1)>, affine_map<(d0, d1, d2, d3) -> (d0, d1, d2, d3)>],\n"
                 "    iterator_types = [\"parallel\", \"parallel\", \"parallel\", \"parallel\"]} "
                 "ins(%x, %b : tensor<1x8x4x5xf32>, tensor<8xf32>) outs(%e : tensor<1x8x4x5xf32>) {\n"
                 "  ^bb0(%a: f32, %c: f32, %o: f32):\n    %s = arith.addf %a, %c : f32\n"
                 "    linalg.yield %s : f32\n  } -> tensor<1x8x4x5xf32>\n"
                 "  return %y : tensor<1x8x4x5xf32>\n}\n")
    h = frontend.nchw_to_nhwc(mlir.parse_functions(bias_text)[0])
    (gen,) = [op for op in h.ops if op.name == "linalg.generic"]
    assert gen.attrs["maps"] == [[0, 1, 2, 3], [3], [0, 1, 2, 3]]
    assert str(h.types["%y"]) == "tensor<1x4x5x8xf32>"


def test_model_zoo_bottleneck_lowers_with_the_final_relu_in_the_residual_conv():
    f = mlir.parse_functions(lower.harness_f32(blocks.model_zoo_bottleneck(2, 256, 64, 56, 56,
                                                                           True)))[0]
    prog = lower.lower(frontend.nchw_to_nhwc(f))
    assert [(c.entry, c.params["act"]) for c in prog.calls] == [
        ("fused_conv2d_nhwc_bias_act", "relu"), ("fused_conv2d_nhwc_bias_act", "relu"),
        ("fused_conv2d_nhwc_bias_res_act", "relu")]


def test_model_zoo_block_lowers_to_three_conv_launches():
    """The block after the harness's f16 -> f32 rule and the layout rewrite:
    expand conv + ReLU, the 3x3 conv with its pad folded + ReLU, the project
    conv with the block input as the residual."""
    f = mlir.parse_functions(lower.harness_f32(blocks.model_zoo_irb(2, 24, 144, 56, 56)))[0]
    prog = lower.lower(frontend.nchw_to_nhwc(f))
    assert [(c.entry, c.params) for c in prog.calls] == [
        ("fused_conv2d_nhwc_bias_act", {"pad": 0, "act": "relu"}),
        ("fused_conv2d_nhwc_bias_act", {"pad": 1, "act": "relu"}),
        ("fused_conv2d_nhwc_bias_res_act", {"pad": 0, "act": "none"})]
    assert prog.calls[2].args[3] == "%x"


class _FloatBottleneck(nn.Module):
    """A ResNet bottleneck without conv biases; BatchNorms that only scale."""

    def __init__(self, C=64, M=64, bn=False):
        super().__init__()
        self.c1 = nn.Conv2d(C, M, 1, bias=False)
        self.c2 = nn.Conv2d(M, M, 3, padding=1, bias=False)
        self.c3 = nn.Conv2d(M, C, 1, bias=False)
        self.bn = bn
        if bn:
            self.b1 = nn.BatchNorm2d(M)
            with torch.no_grad():
                self.b1.weight.uniform_(0.5, 1.5)
                self.b1.running_var.uniform_(0.5, 2.0)
                self.b1.bias.zero_()
                self.b1.running_mean.zero_()

    def forward(self, x):
        y = self.c1(x)
        if self.bn:
            y = self.b1(y)
        y = torch.relu(y)
        y = torch.relu(self.c2(y))
        return torch.relu(self.c3(y) + x)


@pytest.mark.parametrize("bn", [False, True])
def test_int8_frontend_quantizes_a_bottleneck(bn):
    """Post-training quantization of a float bottleneck: the int8 text lowers
    to the int8 bottleneck entry point, and the oracle's int8 result,
    dequantized, follows the float module within the quantization error
    wherever the output is below the output scale's saturation (1.0)."""
    import numpy as np

    import oracle
    torch.manual_seed(1)
    m = _FloatBottleneck(bn=bn)
    x = torch.rand(2, 64, 8, 8)
    text, a = frontend.from_torch_int8(m, x)
    (c,) = lower.lower_text(text).calls
    assert c.entry == "fused_qbottleneck_i8"
    assert a["x"].dtype == np.int8 and a["m1"].dtype == np.int32
    q = oracle.block_qbottleneck(a["x"], a["w1"].reshape(64, 64), a["w2"], a["w3"].reshape(64, 64),
                                 a["m1"], a["s1"], a["m2"], a["s2"], a["m3"], a["s3"])
    fl = m(x).detach().permute(0, 2, 3, 1).numpy()
    ok = fl < 0.99
    assert ok.mean() > 0.9
    assert np.abs(q.astype(np.float64)[ok] / 127 - fl[ok]).max() < 0.05


def test_int8_frontend_refuses_biases_and_other_graphs():
    m = _FloatBottleneck()
    m.c1 = nn.Conv2d(64, 64, 1, bias=True)
    with torch.no_grad():
        m.c1.bias.fill_(0.1)
    with pytest.raises(NotImplementedError, match="bias"):
        frontend.from_torch_int8(m, torch.rand(1, 64, 8, 8))
    with pytest.raises(NotImplementedError, match="bottleneck"):
        frontend.from_torch_int8(nn.Sequential(nn.Conv2d(64, 64, 1, bias=False), nn.ReLU()),
                                 torch.rand(1, 64, 8, 8))
