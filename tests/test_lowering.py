"""Host lowering (npu_amd.lower): linalg text -> entry-point calls.

The outlined names are the reference outliner's (OutlineFusedGroupsPass.cpp:69-82,
259-263), so the groups found here are the groups the reference would call
through its tile loop nests; each becomes one call of the entry point that runs
the whole nest.  What no entry point runs is refused by name, never run
another way.  (The GPU runs of these programs are in test_gpu_parity.py.)
"""

import pytest

import reference_inputs
from npu_amd import blocks, lower, mlir, pipeline



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
    assert c.args == ["%x", "%w", "%bias"]
    # a bf16 bias is widened to f32 exactly before the call (the group adds in f32)
    want = {"pad": pad, "act": "relu", **({"bias_to_f32": True} if elem == "bf16" else {})}
    assert c.params == want


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


@pytest.mark.parametrize("name,calls", [
    ("conv2d_relu.mlir", [("fused_fill_conv2d_generic_0", "fused_conv2d_nchw_bias_act", 1, "relu", 0)]),
    ("resnet_block.mlir", [("fused_fill_conv2d_generic_0", "fused_conv2d_nchw_bias_act", 1, "relu", 0),
                           ("fused_fill_conv2d_generic_1", "fused_conv2d_nchw_bias_res_act", 1,
                            "none", 4)]),
    ("resnet50_block.mlir", [("fused_fill_conv2d_generic_0", "fused_conv2d_nchw_bias_act", 0, "relu", 0),
                             ("fused_fill_conv2d_generic_1", "fused_conv2d_nchw_bias_act", 1, "relu", 0),
                             ("fused_fill_conv2d_generic_generic_2", "fused_conv2d_nchw_bias_res_act",
                              0, "relu", 4)]),
    ("mobilenet_block.mlir", [("fused_fill_conv2d_generic_0", "fused_conv2d_nchw_bias_act", 0, "relu", 0),
                              ("fused_fill_conv2d_generic_1", "fused_conv2d_nchw_bias_act", 1, "relu", 0),
                              ("fused_fill_conv2d_generic_2", "fused_conv2d_nchw_bias_res_act", 0,
                               "none", 4)]),
])
def test_reference_nchw_workloads_lower_to_their_groups(name, calls):
    """The reference's own conv workloads (linalg.conv_2d_nchw_fchw, the
    tensor.pad outside the groups) lower group by group to the NCHW entry
    points under the outliner's names (OutlineFusedGroupsPass.cpp:69-82):
    the pad folded into the launch, a ResNet add (and the ReLU after it, in
    its own generic) as the residual term, named by its argument index."""
    p = lower.lower_text(reference_inputs.read(name))
    got = [(L.name, c.entry, L.pad, L.acts[0], L.res_arg) for L, c in zip(p.launches, p.calls)]
    assert got == calls
    for L, c in zip(p.launches, p.calls):
        if L.res_arg:
            assert L.ins[L.res_arg] == c.args[3] == p.func.args[0][0]


def test_nchw_conv_any_filter_and_stride_lowers():
    """A 5x5 filter and a stride of 2 lower to the NCHW entry point with the
    stride as a launch attribute (the model zoo's 7x7 stems, 9x9 and 5x5
    filters, stride-2 downsampling convs)."""
    t = blocks.nchw_conv_relu(1, 16, 16, 8, 8, elem="f32")
    five = t.replace("16x16x3x3", "16x16x5x5").replace("x10x10xf32", "x12x12xf32") \
        .replace("low[0, 0, 1, 1] high[0, 0, 1, 1]", "low[0, 0, 2, 2] high[0, 0, 2, 2]")
    (L,) = lower.lower_text(five).launches
    assert (L.name, L.pad, L.stride) == ("fused_fill_conv2d_generic_0", 2, 1)
    strided = t.replace("strides = dense<1>", "strides = dense<2>").replace(
        "tensor<1x16x8x8xf32>) -> tensor<1x16x8x8xf32>", "tensor<1x16x8x8xf32>) -> tensor<1x16x4x4xf32>")
    strided = strided.replace("outs(%c_f : tensor<1x16x8x8xf32>) -> tensor<1x16x8x8xf32>",
                              "outs(%c_f : tensor<1x16x4x4xf32>) -> tensor<1x16x4x4xf32>")
    strided = strided.replace("%c_i = tensor.empty() : tensor<1x16x8x8xf32>",
                              "%c_i = tensor.empty() : tensor<1x16x4x4xf32>")
    strided = strided.replace("%c_f = linalg.fill ins(%cst : f32) outs(%c_i : tensor<1x16x8x8xf32>) -> "
                              "tensor<1x16x8x8xf32>", "%c_f = linalg.fill ins(%cst : f32) outs(%c_i : "
                              "tensor<1x16x4x4xf32>) -> tensor<1x16x4x4xf32>")
    (L,) = lower.lower_text(strided).launches
    assert L.stride == 2


def test_nchw_conv_refusals():
    """What the NCHW entry points do not run is refused by name: a dilated
    conv, a pad that is not symmetric in H and W."""
    t = blocks.nchw_conv_relu(1, 16, 16, 8, 8, elem="f32")
    with pytest.raises(NotImplementedError, match="dilated"):
        lower.lower_text(t.replace("dilations = dense<1>", "dilations = dense<2>"))
    lopsided = t.replace("high[0, 0, 1, 1]", "high[0, 0, 1, 2]")
    with pytest.raises(NotImplementedError, match="pad"):
        lower.lower_text(lopsided)


def test_reference_matmul_relu_lowers_through_the_harness_rule():
    """test/matmul_relu.mlir is f16; the reference harness runs it as f32
    (e2e_verify.py:163-164), and so does the lowering: one call, ReLU, no bias."""
    p = lower.lower_text(reference_inputs.read("matmul_relu.mlir"))
    (c,) = p.calls
    assert c.entry == "fused_matmul_bias_act" and c.args == ["%A", "%B", None]
    assert c.params == {"act": "relu"} and c.out == "%relu"
    assert all(t.elem == "f32" for _, t in p.func.args)


def test_reference_mlp_is_two_calls():
    """test/mlp.mlir outlines as one group of two matmul -> ReLU chains; it
    runs as two calls, the second reading the first's result."""
    p = lower.lower_text(reference_inputs.read("mlp.mlir"))
    assert [c.entry for c in p.calls] == ["fused_matmul_bias_act"] * 2
    assert p.calls[0].args == ["%input", "%w1", None] and p.calls[0].out == "%relu1"
    assert p.calls[1].args == ["%relu1", "%w2", None] and p.calls[1].out == "%relu2"
    assert p.calls[0].functions == p.calls[1].functions


def _shape_of(func):
    """The function with SSA names replaced by first-appearance numbers: op
    names, operand/result types, indexing maps, iterators, generic bodies,
    pad widths and strides."""
    ids = {}

    def n(v):
        return ids.setdefault(v, f"v{len(ids)}")
    for a, _ in func.args:
        n(a)
    out = [[str(t) for _, t in func.args], [str(t) for t in func.result_types]]
    for op in func.ops:
        if op.name == "tensor.empty":
            continue  # placeholders: the builder names one per generic
        for r in op.results:
            n(r)
        body = [(b.name, b.value) for b in op.attrs.get("body", [])]
        out.append((op.name, [n(v) for v in op.ins + op.operands if v in ids],
                    [str(func.types[r]) for r in op.results], op.attrs.get("maps"),
                    op.iterators, body, op.attrs.get("value"), op.attrs.get("low"),
                    op.attrs.get("high"), op.attrs.get("strides")))
    return out


@pytest.mark.parametrize("name", ["matmul_relu.mlir", "mlp.mlir", "conv2d_relu.mlir",
                                  "resnet_block.mlir", "resnet50_block.mlir",
                                  "mobilenet_block.mlir"])
def test_builder_text_is_the_reference_workload(name):
    """The GPU box has no reference checkout, so the GPU runs the builder's
    text of these workloads; here it is checked against the reference's file."""
    ref = mlir.parse_functions(reference_inputs.read(name))[0]
    own = mlir.parse_functions(blocks.reference_workload(name))[0]
    assert _shape_of(own) == _shape_of(ref)


def _replace_body(text, old, new):
    assert old in text
    return text.replace(old, new)


def test_bias_through_mulf_is_refused():
    t = _replace_body(blocks.matmul_bias_act(8, 16, 8), "%s0 = arith.addf %in, %b",
                      "%s0 = arith.mulf %in, %b")
    with pytest.raises(NotImplementedError, match="arith.mulf"):
        lower.lower_text(t)


def test_bias_on_the_row_dimension_is_refused():
    t = _replace_body(blocks.matmul_bias_act(8, 16, 8), "affine_map<(d0, d1) -> (d1)>",
                      "affine_map<(d0, d1) -> (d0)>")
    with pytest.raises(NotImplementedError, match="map"):
        lower.lower_text(t)


def test_nonzero_fill_and_clamp_are_refused():
    t = _replace_body(blocks.matmul_bias_act(8, 16, 8), "%cst = arith.constant 0.0 : f32",
                      "%cst = arith.constant 1.0 : f32")
    with pytest.raises(NotImplementedError, match="fill"):
        lower.lower_text(t)
    t = _replace_body(blocks.matmul_bias_act(8, 16, 8), "%z = arith.constant 0.0 : f32",
                      "%z = arith.constant 3.0 : f32")
    with pytest.raises(NotImplementedError):
        lower.lower_text(t)


def test_relu6_bound_and_order_are_checked():
    t = _replace_body(blocks.matmul_bias_act(8, 16, 8, act="relu6"),
                      "%six = arith.constant 6.0 : f32", "%six = arith.constant 5.0 : f32")
    with pytest.raises(NotImplementedError):
        lower.lower_text(t)


def test_output_block_argument_is_refused():
    """Reading the generic's `outs` block argument accumulates into the
    destination, which no entry point does."""
    t = _replace_body(blocks.matmul_bias_act(8, 16, 8), "%s0 = arith.addf %in, %b",
                      "%s0 = arith.addf %in, %out")
    with pytest.raises(NotImplementedError, match="block argument"):
        lower.lower_text(t)


def test_nonzero_pad_is_refused():
    t = blocks.conv_bias_act(1, 8, 8, 16, 16)
    t = _replace_body(t, "tensor.yield %cst : f32", "tensor.yield %one : f32")
    t = _replace_body(t, "%cst = arith.constant 0.0 : f32\n",
                      "%cst = arith.constant 0.0 : f32\n  %one = arith.constant 1.0 : f32\n")
    with pytest.raises(NotImplementedError, match="pad"):
        lower.lower_text(t)


def test_dilated_conv_is_refused():
    t = _replace_body(blocks.conv_bias_act(1, 8, 8, 16, 16, pad=0), "dilations = dense<1>",
                      "dilations = dense<2>")
    with pytest.raises(NotImplementedError, match="dilated"):
        lower.lower_text(t)


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


def test_program_checks_inputs_against_the_signature():
    import torch
    p = lower.lower_text(blocks.matmul_bias_act(8, 16, 4))
    ok = {"A": torch.zeros(8, 16), "B": torch.zeros(16, 4), "bias": torch.zeros(4)}
    assert set(p.check_inputs(ok)) == {"%A", "%B", "%bias"}
    with pytest.raises(TypeError, match="%bias"):
        p.check_inputs(dict(ok, bias=torch.zeros(4, dtype=torch.bfloat16)))
    with pytest.raises(ValueError, match="%B"):
        p.check_inputs(dict(ok, B=torch.zeros(4, 16)))
    with pytest.raises(KeyError):
        p.check_inputs({"A": ok["A"]})


def test_pipeline_names_entry_points_without_the_hip_library():
    from npu_amd import names
    rep = pipeline.run(mlir.parse_functions(blocks.matmul_bias_act(8, 16, 4))[0])
    assert rep["functions"][0]["entry_point"] == "fused_matmul_bias_act"
    assert names.OUTLINED_NAMES["fused_fill_matmul_generic"] == "fused_matmul_bias_act"


def test_int8_bottleneck_lowers_to_one_call():
    """The int8 bottleneck text (apply_scale requant generics, a zero pad
    before the 3x3 conv, the residual in the last generic) outlines as two
    groups around the pad and runs as one fused_qbottleneck_i8 launch."""
    p = lower.lower_text(blocks.qbottleneck(2, 7, 9, 64, 64))
    (c,) = p.calls
    assert c.entry == "fused_qbottleneck_i8" and len(c.functions) == 2
    assert c.args == ["%x", "%w1", "%w2", "%w3", "%m1", "%s1", "%m2", "%s2", "%m3", "%s3"]
    assert c.views == {"%w1": [64, 64], "%w3": [64, 64]}
    (L,) = p.launches
    assert L.name == "+".join(c.functions) and len(L.ins) == 17 and "%y1p" not in L.ins


@pytest.mark.parametrize("old,new", [
    ("%rnd = arith.shli %one, %sm1 : i64", "%rnd = arith.shli %one, %s64 : i64"),  # wrong rounding
    ("%q = arith.shrsi %t, %s64 : i64", "%q = arith.shrui %t, %s64 : i64"),     # logical shift
    ("%hi = arith.constant 127 : i32", "%hi = arith.constant 100 : i32"),       # clamp bound
    ("%p = arith.muli %a64, %m64 : i64", "%p = arith.addi %a64, %m64 : i64"),   # not a product
])
def test_int8_requant_bodies_are_checked(old, new):
    t = blocks.qbottleneck(1, 4, 4, 64, 64)
    assert old in t
    with pytest.raises(NotImplementedError):
        lower.lower_text(t.replace(old, new, 1))


def test_int8_residual_must_be_the_input():
    t = blocks.qbottleneck(1, 4, 4, 64, 64).replace("ins(%acc3, %m3, %s3, %x :", "ins(%acc3, %m3, %s3, %y2 :")
    with pytest.raises(NotImplementedError):
        lower.lower_text(t)


def test_llama_layer_lowers_to_the_four_entry_points():
    """The Llama decoder layer in linalg (RMSNorm, RoPE on interleaved pairs,
    causal softmax attention over per-head views, residual projections,
    SwiGLU) outlines into ten groups; the matcher follows the dataflow and
    runs it as five calls of the four Llama entry points."""
    p = lower.lower_text(blocks.llama_layer(64, 128, 2, 192))
    got = [(c.entry, c.args, c.outs, c.params) for c in p.calls]
    assert got == [
        ("fused_llama_qkv_rope", ["%x", "%g1", "%wq", "%wk", "%wv", "%cos", "%sin"],
         ["%Q", "%K", "%V"], {"eps": 1e-05}),
        ("fused_llama_attention", ["%Q", "%K", "%V"], ["%A"], {"n_heads": 2, "scale": 0.125}),
        ("fused_llama_matmul_residual", ["%A", "%wo", "%x"], ["%h"], {}),
        ("fused_llama_rmsnorm_swiglu", ["%h", "%g2", "%wg", "%wu"], ["%act"], {"eps": 1e-05}),
        ("fused_llama_matmul_residual", ["%act", "%wd", "%h"], ["%out"], {}),
    ]
    assert [L.entry for L in p.launches] == [c.entry for c in p.calls]
    assert all(n.startswith("fused_") for c in p.calls for n in c.functions)


def test_llama_roles_follow_the_attention_views():
    """Which rotated projection is the query is read from the attention's
    views (Q: [1, 0, 2], K: [1, 2, 0]), not from the order of the matmuls."""
    t = blocks.llama_layer(64, 128, 2, 192)
    t = t.replace("%A_q_3 = tensor.expand_shape %Q ", "%A_q_3 = tensor.expand_shape %TMP ")
    t = t.replace("%A_k_3 = tensor.expand_shape %K ", "%A_k_3 = tensor.expand_shape %Q ")
    t = t.replace("%A_q_3 = tensor.expand_shape %TMP ", "%A_q_3 = tensor.expand_shape %K ")
    c = lower.lower_text(t).calls[0]
    assert c.args[2:4] == ["%wk", "%wq"] and c.outs == ["%K", "%Q", "%V"]


@pytest.mark.parametrize("old,new", [
    # RMSNorm: x * (inv * g) is another rounding than (x * inv) * g
    ("%t = arith.mulf %e, %inv : f32\n    %u = arith.mulf %t, %g : f32",
     "%t = arith.mulf %inv, %g : f32\n    %u = arith.mulf %e, %t : f32"),
    ("%d = arith.constant 128.0 : f32", "%d = arith.constant 64.0 : f32"),     # mean over D
    ("%ev = arith.subf %a, %b : f32", "%ev = arith.addf %a, %b : f32"),          # rotation sign
    ("%is0 = arith.cmpi eq, %j, %c0 : index", "%is0 = arith.cmpi ne, %j, %c0 : index"),
    ("%gt = arith.cmpi ugt, %j, %i : index", "%gt = arith.cmpi uge, %j, %i : index"),  # diagonal
    ("%d = arith.subf %a, %m : f32", "%d = arith.subf %m, %a : f32"),            # exp(m - s)
    ("%m = arith.maximumf %acc, %a : f32", "%m = arith.minimumf %acc, %a : f32"),
    ("%s = arith.divf %g, %den : f32", "%s = arith.mulf %g, %den : f32"),          # not SiLU
    ("%s = arith.addf %e, %a : f32", "%s = arith.subf %e, %a : f32"),             # residual
])
def test_llama_bodies_are_checked(old, new):
    t = blocks.llama_layer(64, 128, 2, 192)
    assert old in t
    with pytest.raises(NotImplementedError):
        lower.lower_text(t.replace(old, new, 1))


def test_llama_views_and_head_size_are_checked():
    t = blocks.llama_layer(64, 128, 2, 192)
    # K viewed like Q (no transpose of the key) is not Q K^T
    bad = t.replace("permutation = [1, 2, 0]", "permutation = [1, 0, 2]", 1)
    with pytest.raises(NotImplementedError):
        lower.lower_text(bad)
    # heads of 32: the attention entry point's head dimensions are 64 and 128
    with pytest.raises(NotImplementedError, match="head dimensions are 64 and 128"):
        lower.lower_text(blocks.llama_layer(64, 128, 4, 192, dh=32))
    # heads of 128 lower to the same five calls
    prog = lower.lower_text(blocks.llama_layer(64, 256, 2, 192, dh=128))
    assert prog.entry_points == ["fused_llama_qkv_rope", "fused_llama_attention",
                                 "fused_llama_matmul_residual", "fused_llama_rmsnorm_swiglu",
                                 "fused_llama_matmul_residual"]
