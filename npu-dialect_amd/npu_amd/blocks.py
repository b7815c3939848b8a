"""linalg text of the fused blocks, for the lowering (npu_amd.lower) and its tests.

The reference generates its model inputs as MLIR text (tools/gen_model_mlir.py,
NCHW f16); these are the NHWC blocks the MI355X entry points execute, written the
way the reference writes its own: `tensor.pad` with a zero yield, a
`linalg.fill` init, the named op, and a `linalg.generic` epilogue whose body
holds the bias add and the activation (`arith.maximumf` with 0 for ReLU, then
`arith.minimumf` with 6 for ReLU6, as test/mobilenet_block.mlir:26-36 does).
"""
from __future__ import annotations


def _t(shape, elem):
    return "tensor<" + "x".join(str(d) for d in shape) + "x" + elem + ">"


def _maps(rank, bias):
    ids = ", ".join(f"d{i}" for i in range(rank))
    full = f"affine_map<({ids}) -> ({ids})>"
    if not bias:
        return f"[{full}, {full}]"
    return f"[{full}, affine_map<({ids}) -> (d{rank - 1})>, {full}]"


def _epilogue(res, src, bias, shape, elem, act, residual=None):
    """`res` = act(src [+ bias] [+ residual]) as one linalg.generic."""
    rank = len(shape)
    ins, tys, args, lines = [src], [_t(shape, elem)], ["%in: " + elem], []
    maps = []
    ids = ", ".join(f"d{i}" for i in range(rank))
    full = f"affine_map<({ids}) -> ({ids})>"
    maps.append(full)
    v = "%in"
    if bias is not None:
        ins.append(bias)
        tys.append(_t([shape[-1]], elem))
        args.append("%b: " + elem)
        maps.append(f"affine_map<({ids}) -> (d{rank - 1})>")
        lines.append(f"    %s0 = arith.addf {v}, %b : {elem}")
        v = "%s0"
    if residual is not None:
        ins.append(residual)
        tys.append(_t(shape, elem))
        args.append("%r: " + elem)
        maps.append(full)
        lines.append(f"    %s1 = arith.addf {v}, %r : {elem}")
        v = "%s1"
    maps.append(full)
    if act in ("relu", "relu6"):
        lines.append(f"    %z = arith.constant 0.0 : {elem}")
        lines.append(f"    %a0 = arith.maximumf {v}, %z : {elem}")
        v = "%a0"
    if act == "relu6":
        lines.append(f"    %six = arith.constant 6.0 : {elem}")
        lines.append(f"    %a1 = arith.minimumf {v}, %six : {elem}")
        v = "%a1"
    if act not in ("none", "relu", "relu6"):
        raise ValueError(f"unknown activation {act!r}")
    it = ", ".join(['"parallel"'] * rank)
    return (f"  {res}_e = tensor.empty() : {_t(shape, elem)}\n"
            f"  {res} = linalg.generic {{indexing_maps = [{', '.join(maps)}],\n"
            f"    iterator_types = [{it}]}} ins({', '.join(ins)} : {', '.join(tys)}) "
            f"outs({res}_e : {_t(shape, elem)}) {{\n"
            f"  ^bb0({', '.join(args)}, %out: {elem}):\n" + "\n".join(lines) +
            f"\n    linalg.yield {v} : {elem}\n  }} -> {_t(shape, elem)}\n")


def matmul_bias_act(M, K, N, act="relu", bias=True, elem="f32"):
    """C1: out[M,N] = act(A[M,K] @ B[K,N] + bias[N])."""
    b = f", %bias: {_t([N], elem)}" if bias else ""
    return (f"func.func @matmul_bias_act(%A: {_t([M, K], elem)}, %B: {_t([K, N], elem)}{b}) -> "
            f"{_t([M, N], elem)} {{\n"
            f"  %cst = arith.constant 0.0 : {elem}\n"
            f"  %init = tensor.empty() : {_t([M, N], elem)}\n"
            f"  %fill = linalg.fill ins(%cst : {elem}) outs(%init : {_t([M, N], elem)}) -> "
            f"{_t([M, N], elem)}\n"
            f"  %mm = linalg.matmul ins(%A, %B : {_t([M, K], elem)}, {_t([K, N], elem)}) "
            f"outs(%fill : {_t([M, N], elem)}) -> {_t([M, N], elem)}\n" +
            _epilogue("%y", "%mm", "%bias" if bias else None, [M, N], elem, act) +
            f"  return %y : {_t([M, N], elem)}\n}}\n")


def _conv(res, x, w, xshape, wshape, oshape, elem, name="linalg.conv_2d_nhwc_fhwc"):
    return (f"  {res}_i = tensor.empty() : {_t(oshape, elem)}\n"
            f"  {res}_f = linalg.fill ins(%cst : {elem}) outs({res}_i : {_t(oshape, elem)}) -> "
            f"{_t(oshape, elem)}\n"
            f"  {res} = {name} {{dilations = dense<1> : tensor<2xi64>, "
            f"strides = dense<1> : tensor<2xi64>}}\n"
            f"    ins({x}, {w} : {_t(xshape, elem)}, {_t(wshape, elem)}) "
            f"outs({res}_f : {_t(oshape, elem)}) -> {_t(oshape, elem)}\n")


def _pad(res, x, shape, p, elem):
    padded = [shape[0], shape[1] + 2 * p, shape[2] + 2 * p, shape[3]]
    return (f"  {res} = tensor.pad {x} low[0, {p}, {p}, 0] high[0, {p}, {p}, 0] {{\n"
            f"  ^bb0(%i0: index, %i1: index, %i2: index, %i3: index):\n"
            f"    tensor.yield %cst : {elem}\n"
            f"  }} : {_t(shape, elem)} to {_t(padded, elem)}\n"), padded


def conv_bias_act(N, H, W, C, F, K=3, pad=1, act="relu", bias=True, elem="f32"):
    """C2: out = act(conv_2d_nhwc_fhwc(pad(x), w[F,K,K,C]) + bias[F])."""
    Ho, Wo = H + 2 * pad - K + 1, W + 2 * pad - K + 1
    b = f", %bias: {_t([F], elem)}" if bias else ""
    text = (f"func.func @conv_bias_act(%x: {_t([N, H, W, C], elem)}, "
            f"%w: {_t([F, K, K, C], elem)}{b}) -> {_t([N, Ho, Wo, F], elem)} {{\n"
            f"  %cst = arith.constant 0.0 : {elem}\n")
    xin, xshape = "%x", [N, H, W, C]
    if pad:
        t, xshape = _pad("%xp", "%x", [N, H, W, C], pad, elem)
        text += t
        xin = "%xp"
    text += _conv("%conv", xin, "%w", xshape, [F, K, K, C], [N, Ho, Wo, F], elem)
    text += _epilogue("%y", "%conv", "%bias" if bias else None, [N, Ho, Wo, F], elem, act)
    return text + f"  return %y : {_t([N, Ho, Wo, F], elem)}\n}}\n"


def inverted_residual(N, H, W, C, E, elem="f32"):
    """C3 (MobileNetV2 inverted residual, NHWC, no BN): expand 1x1 + ReLU6,
    pad, depthwise 3x3 + ReLU6, project 1x1, + x."""
    xs, es = [N, H, W, C], [N, H, W, E]
    text = (f"func.func @inverted_residual(%x: {_t(xs, elem)}, %we: {_t([E, 1, 1, C], elem)}, "
            f"%wdw: {_t([3, 3, E], elem)}, %wp: {_t([C, 1, 1, E], elem)}) -> {_t(xs, elem)} {{\n"
            f"  %cst = arith.constant 0.0 : {elem}\n")
    text += _conv("%ex", "%x", "%we", xs, [E, 1, 1, C], es, elem)
    text += _epilogue("%e", "%ex", None, es, elem, "relu6")
    t, ps = _pad("%ep", "%e", es, 1, elem)
    text += t
    text += _conv("%dw", "%ep", "%wdw", ps, [3, 3, E], es, elem,
                  name="linalg.depthwise_conv_2d_nhwc_hwc")
    text += _epilogue("%d", "%dw", None, es, elem, "relu6")
    text += _conv("%pr", "%d", "%wp", es, [C, 1, 1, E], xs, elem)
    text += _epilogue("%y", "%pr", None, xs, elem, "none", residual="%x")
    return text + f"  return %y : {_t(xs, elem)}\n}}\n"


def mlp(M, K, H, N, elem="f32"):
    """Two matmul -> ReLU layers, out = relu(relu(x @ w1) @ w2): the workload of
    test/mlp.mlir (128x256 . 256x512 . 512x256 in f16 there), written by this
    builder with the same ops, types and generic bodies."""
    def layer(i, x, w, xs, ws, os_):
        return (f"  %init{i} = tensor.empty() : {_t(os_, elem)}\n"
                f"  %fill{i} = linalg.fill ins(%cst : {elem}) outs(%init{i} : {_t(os_, elem)}) -> "
                f"{_t(os_, elem)}\n"
                f"  %mm{i} = linalg.matmul ins({x}, {w} : {_t(xs, elem)}, {_t(ws, elem)}) "
                f"outs(%fill{i} : {_t(os_, elem)}) -> {_t(os_, elem)}\n" +
                _epilogue(f"%relu{i}", f"%mm{i}", None, os_, elem, "relu"))
    return (f"func.func @mlp(%input: {_t([M, K], elem)}, %w1: {_t([K, H], elem)}, "
            f"%w2: {_t([H, N], elem)}) -> {_t([M, N], elem)} {{\n"
            f"  %cst = arith.constant 0.0 : {elem}\n" +
            layer(1, "%input", "%w1", [M, K], [K, H], [M, H]) +
            layer(2, "%relu1", "%w2", [M, H], [H, N], [M, N]) +
            f"  return %relu2 : {_t([M, N], elem)}\n}}\n")


def reference_workload(name):
    """Builder text of a reference test workload, by its file name:
    test/matmul_relu.mlir (fill -> matmul 128x256 . 256x512 -> ReLU, f16) and
    test/mlp.mlir.  They run on the GPU where the reference's files are not
    present; a CPU test checks that each has the same ops, types, indexing maps
    and generic bodies as the reference's file."""
    if name == "matmul_relu.mlir":
        return matmul_bias_act(128, 256, 512, act="relu", bias=False, elem="f16")
    if name == "mlp.mlir":
        return mlp(128, 256, 512, 256, elem="f16")
    raise KeyError(name)


def _requant(res, acc, m, s, shape, residual=None):
    """`res` (i8) = clamp(apply_scale(acc) [+ residual], 0, 127) as one
    linalg.generic: TOSA apply_scale_32 with single rounding written in arith
    -- (i64(acc) * i64(m) + (1 << (s - 1))) >> s, truncated to i32 -- then
    the residual added in i32, the clamp (ReLU folded into [0, 127]) and the
    truncation to i8.  m and s are per output channel (the last dimension)."""
    rank = len(shape)
    ids = ", ".join(f"d{i}" for i in range(rank))
    full, chan = f"affine_map<({ids}) -> ({ids})>", f"affine_map<({ids}) -> (d{rank - 1})>"
    ins, tys, maps, args = [acc, m, s], [_t(shape, "i32"), _t([shape[-1]], "i32"),
                                         _t([shape[-1]], "i32")], [full, chan, chan], \
        ["%a: i32", "%m: i32", "%s: i32"]
    if residual is not None:
        ins.append(residual)
        tys.append(_t(shape, "i8"))
        maps.append(full)
        args.append("%x: i8")
    maps.append(full)
    body = ["    %a64 = arith.extsi %a : i32 to i64",
            "    %m64 = arith.extsi %m : i32 to i64",
            "    %s64 = arith.extsi %s : i32 to i64",
            "    %p = arith.muli %a64, %m64 : i64",
            "    %one = arith.constant 1 : i64",
            "    %sm1 = arith.subi %s64, %one : i64",
            "    %rnd = arith.shli %one, %sm1 : i64",
            "    %t = arith.addi %p, %rnd : i64",
            "    %q = arith.shrsi %t, %s64 : i64",
            "    %q32 = arith.trunci %q : i64 to i32"]
    v = "%q32"
    if residual is not None:
        body += ["    %x32 = arith.extsi %x : i8 to i32", "    %r = arith.addi %q32, %x32 : i32"]
        v = "%r"
    body += ["    %lo = arith.constant 0 : i32", "    %hi = arith.constant 127 : i32",
             f"    %c1 = arith.maxsi {v}, %lo : i32", "    %c2 = arith.minsi %c1, %hi : i32",
             "    %o = arith.trunci %c2 : i32 to i8"]
    it = ", ".join(['"parallel"'] * rank)
    return (f"  {res}_e = tensor.empty() : {_t(shape, 'i8')}\n"
            f"  {res} = linalg.generic {{indexing_maps = [{', '.join(maps)}],\n"
            f"    iterator_types = [{it}]}} ins({', '.join(ins)} : {', '.join(tys)}) "
            f"outs({res}_e : {_t(shape, 'i8')}) {{\n"
            f"  ^bb0({', '.join(args)}, %out: i8):\n" + "\n".join(body) +
            f"\n    linalg.yield %o : i8\n  }} -> {_t(shape, 'i8')}\n")


def _iconv(res, x, w, xshape, wshape, oshape, zero="%c0"):
    return (f"  {res}_i = tensor.empty() : {_t(oshape, 'i32')}\n"
            f"  {res}_f = linalg.fill ins({zero} : i32) outs({res}_i : {_t(oshape, 'i32')}) -> "
            f"{_t(oshape, 'i32')}\n"
            f"  {res} = linalg.conv_2d_nhwc_fhwc {{dilations = dense<1> : tensor<2xi64>, "
            f"strides = dense<1> : tensor<2xi64>}}\n"
            f"    ins({x}, {w} : {_t(xshape, 'i8')}, {_t(wshape, 'i8')}) "
            f"outs({res}_f : {_t(oshape, 'i32')}) -> {_t(oshape, 'i32')}\n")


def qbottleneck(N, H, W, C, M1):
    """C4 (int8 ResNet-50 bottleneck, NHWC, zero points 0): 1x1 C -> M1,
    requant + ReLU; pad; 3x3 M1 -> M1, requant + ReLU; 1x1 M1 -> C, requant,
    + x, ReLU (the int8 restatement of test/resnet50_block.mlir:5-105)."""
    xs, ys = [N, H, W, C], [N, H, W, M1]
    ps = [N, H + 2, W + 2, M1]
    sig = (f"%x: {_t(xs, 'i8')}, %w1: {_t([M1, 1, 1, C], 'i8')}, %w2: {_t([M1, 3, 3, M1], 'i8')}, "
           f"%w3: {_t([C, 1, 1, M1], 'i8')}, %m1: {_t([M1], 'i32')}, %s1: {_t([M1], 'i32')}, "
           f"%m2: {_t([M1], 'i32')}, %s2: {_t([M1], 'i32')}, %m3: {_t([C], 'i32')}, "
           f"%s3: {_t([C], 'i32')}")
    text = (f"func.func @qbottleneck({sig}) -> {_t(xs, 'i8')} {{\n"
            f"  %c0 = arith.constant 0 : i32\n  %z8 = arith.constant 0 : i8\n")
    text += _iconv("%acc1", "%x", "%w1", xs, [M1, 1, 1, C], ys)
    text += _requant("%y1", "%acc1", "%m1", "%s1", ys)
    text += (f"  %y1p = tensor.pad %y1 low[0, 1, 1, 0] high[0, 1, 1, 0] {{\n"
             f"  ^bb0(%i0: index, %i1: index, %i2: index, %i3: index):\n"
             f"    tensor.yield %z8 : i8\n  }} : {_t(ys, 'i8')} to {_t(ps, 'i8')}\n")
    text += _iconv("%acc2", "%y1p", "%w2", ps, [M1, 3, 3, M1], ys)
    text += _requant("%y2", "%acc2", "%m2", "%s2", ys)
    text += _iconv("%acc3", "%y2", "%w3", ys, [C, 1, 1, M1], xs)
    text += _requant("%y3", "%acc3", "%m3", "%s3", xs, residual="%x")
    return text + f"  return %y3 : {_t(xs, 'i8')}\n}}\n"
