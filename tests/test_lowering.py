"""Host lowering (npu_amd.lower): linalg text -> entry-point calls.

The outlined names are the reference outliner's (OutlineFusedGroupsPass.cpp:69-82,
259-263), so the groups found here are the groups the reference would call
through its tile loop nests; each becomes one call of the entry point that runs
the whole nest.  What no entry point runs is refused by name, never run
another way.  (The GPU runs of these programs are in test_gpu_parity.py.)
"""
import os

import pytest

from npu_amd import blocks, lower, mlir, pipeline

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "mlir")


def test_matmul_bias_act_is_one_call():
    p = lower.lower_text(blocks.matmul_bias_act(64, 128, 32, act="relu"))
    (c,) = p.calls
    assert c.entry == "fused_matmul_bias_act" and c.functions == ["fused_fill_matmul_generic_0"]
    assert c.args == ["%A", "%B", "%bias"] and c.out == "%y" and c.params == {"act": "relu"}
    (c,) = lower.lower_text(blocks.matmul_bias_act(64, 128, 32, act="relu6", bias=False)).calls
    assert c.args == ["%A", "%B", None] and c.params == {"act": "relu6"}
    (c,) = lower.lower_text(blocks.matmul_bias_act(8, 16, 8, act="none")).calls
    assert c.params == {"act": "none"}


@pytest.mark.parametrize("K,pad,elem", [(3, 1, "f32"), (3, 0, "bf16"), (1, 0, "f32")])
def test_conv_folds_the_pad(K, pad, elem):
    p = lower.lower_text(blocks.conv_bias_act(2, 8, 8, 16, 32, K=K, pad=pad, elem=elem))
    (c,) = p.calls
    assert c.entry == "fused_conv2d_nhwc_bias_act"
    assert c.functions == ["fused_fill_linalg_conv_2d_nhwc_fhwc_generic_0"]
    assert c.args == ["%x", "%w", "%bias"] and c.params == {"pad": pad, "act": "relu"}


@pytest.mark.parametrize("shape,ngroups", [((1, 8, 8, 24, 144), 2), ((2, 9, 13, 24, 144), 3)])
def test_inverted_residual_chain_is_one_call(shape, ngroups):
    """Expand (1x1 + ReLU6), pad, depthwise + ReLU6, project, + x: outlined as
    two groups and a pad, or three when the fusion decision (cost-model
    driven) keeps the depthwise apart, and run as one fused_irb_f32 call; the
    filters are viewed without their unit dimensions."""
    text = blocks.inverted_residual(*shape)
    rep = pipeline.run(mlir.parse_functions(text)[0])
    assert len(rep["functions"]) == ngroups
    if ngroups == 2:
        assert [f["entry_point"] for f in rep["functions"]] == ["fused_conv2d_nhwc_bias_act",
                                                               "fused_irb_f32"]
    (c,) = lower.lower_text(text).calls
    assert c.entry == "fused_irb_f32" and len(c.functions) == ngroups
    assert c.args == ["%x", "%we", "%wdw", "%wp"] and c.out == "%y"
    assert c.views == {"%we": [144, 24], "%wp": [24, 144]}


@pytest.mark.parametrize("path,what", [
    ("mlp.mlir", "no MI355X entry point"),        # matmul -> relu -> matmul -> relu, one group
    ("conv2d_relu.mlir", "no MI355X entry point"),  # NCHW convolution
    ("matmul_relu.mlir", "element type f16"),
])
def test_unsupported_is_refused(path, what):
    f = mlir.parse_file(os.path.join(GOLD, path))[0]
    with pytest.raises(NotImplementedError, match=what):
        lower.lower(f)


def test_strided_and_asymmetric_pads_are_refused():
    t = blocks.conv_bias_act(1, 8, 8, 16, 16).replace(
        "strides = dense<1> : tensor<2xi64>", "strides = dense<2> : tensor<2xi64>")
    with pytest.raises(NotImplementedError, match="strided"):
        lower.lower_text(t)
    t = blocks.conv_bias_act(1, 8, 8, 16, 16).replace("high[0, 1, 1, 0]", "high[0, 2, 2, 0]")
    t = t.replace("to tensor<1x10x10x16xf32>", "to tensor<1x11x11x16xf32>").replace(
        "tensor<1x10x10x16xf32>, tensor<16x3x3x16xf32>", "tensor<1x11x11x16xf32>, tensor<16x3x3x16xf32>")
    with pytest.raises(NotImplementedError, match="pad"):
        lower.lower_text(t)
