"""linalg text of the fused blocks, for the lowering (npu_amd.lower) and its tests.

The reference generates its model inputs as MLIR text (tools/gen_model_mlir.py,
NCHW f16); these are the NHWC blocks the MI355X entry points execute, written the
way the reference writes its own: `tensor.pad` with a zero yield, a
`linalg.fill` init, the named op, and a `linalg.generic` epilogue whose body
holds the bias add and the activation (`arith.maximumf` with 0 for ReLU, then
`arith.minimumf` with 6 for ReLU6, as test/mobilenet_block.mlir:26-36 does).
"""
from __future__ import annotations

import math


def _t(shape, elem):
    return "tensor<" + "x".join(str(d) for d in shape) + "x" + elem + ">"


def _maps(rank, bias):
    ids = ", ".join(f"d{i}" for i in range(rank))
    full = f"affine_map<({ids}) -> ({ids})>"
    if not bias:
        return f"[{full}, {full}]"
    return f"[{full}, affine_map<({ids}) -> (d{rank - 1})>, {full}]"


def _epilogue(res, src, bias, shape, elem, act, residual=None, bias_dim=None):
    """`res` = act(src [+ bias] [+ residual]) as one linalg.generic; the bias
    runs along dimension `bias_dim` (default the last)."""
    rank = len(shape)
    bias_dim = rank - 1 if bias_dim is None else bias_dim
    ins, tys, args, lines = [src], [_t(shape, elem)], ["%in: " + elem], []
    maps = []
    ids = ", ".join(f"d{i}" for i in range(rank))
    full = f"affine_map<({ids}) -> ({ids})>"
    maps.append(full)
    v = "%in"
    if bias is not None:
        ins.append(bias)
        tys.append(_t([shape[bias_dim]], elem))
        args.append("%b: " + elem)
        maps.append(f"affine_map<({ids}) -> (d{bias_dim})>")
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
    test/matmul_relu.mlir (fill -> matmul 128x256 . 256x512 -> ReLU, f16),
    test/mlp.mlir and the NCHW conv workloads test/conv2d_relu.mlir,
    test/resnet_block.mlir, test/resnet50_block.mlir and
    test/mobilenet_block.mlir (f16 text, conv_2d_nchw_fchw).  They run on the GPU where the reference's files are not
    present; a CPU test checks that each has the same ops, types, indexing maps
    and generic bodies as the reference's file."""
    if name == "matmul_relu.mlir":
        return matmul_bias_act(128, 256, 512, act="relu", bias=False, elem="f16")
    if name == "mlp.mlir":
        return mlp(128, 256, 512, 256, elem="f16")
    if name == "conv2d_relu.mlir":
        return nchw_conv_relu(1, 64, 64, 56, 56)
    if name == "resnet_block.mlir":
        return nchw_resnet_block(1, 64, 56, 56)
    if name == "resnet50_block.mlir":
        return model_zoo_bottleneck(1, 256, 64, 56, 56, True, name="resnet50_block")
    if name == "mobilenet_block.mlir":
        return model_zoo_bottleneck(1, 32, 192, 112, 112, False, name="mobilenet_block")
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


def _gen(res, ins, in_types, out_elem, out_shape, maps, iters, args, body, yielded, init=None):
    """One linalg.generic, its destination a tensor.empty (or `init`)."""
    it = ", ".join(f'"{x}"' for x in iters)
    dest = init or f"{res}_e"
    pre = "" if init else f"  {res}_e = tensor.empty() : {_t(out_shape, out_elem)}\n"
    return (pre + f"  {res} = linalg.generic {{indexing_maps = [{', '.join(maps)}],\n"
            f"    iterator_types = [{it}]}} ins({', '.join(ins)} : {', '.join(in_types)}) "
            f"outs({dest} : {_t(out_shape, out_elem)}) {{\n"
            f"  ^bb0({', '.join(args)}):\n" + "\n".join("    " + b for b in body) +
            f"\n    linalg.yield {yielded} : {out_elem}\n  }} -> {_t(out_shape, out_elem)}\n")


def _amap(n, res):
    ids = ", ".join(f"d{i}" for i in range(n))
    return f"affine_map<({ids}) -> ({res})>"


def _fill(res, shape, elem, value):
    return (f"  {res}_i = tensor.empty() : {_t(shape, elem)}\n"
            f"  {res} = linalg.fill ins({value} : {elem}) outs({res}_i : {_t(shape, elem)}) -> "
            f"{_t(shape, elem)}\n")


def _rmsnorm(res, x, g, S, D, eps):
    """res (bf16) = bf16(x * (1 / sqrt(sum(x^2) / D + eps)) * g), the sum of
    squares a reduction generic over the row."""
    idd, row, col = _amap(2, "d0, d1"), _amap(2, "d0"), _amap(2, "d1")
    t = _fill(f"{res}_ss0", [S], "f32", "%zf")
    t += _gen(f"{res}_ss", [x], [_t([S, D], "bf16")], "f32", [S], [idd, row],
              ["parallel", "reduction"], ["%a: bf16", "%acc: f32"],
              ["%e = arith.extf %a : bf16 to f32", "%q = arith.mulf %e, %e : f32",
               "%s = arith.addf %acc, %q : f32"], "%s", init=f"{res}_ss0")
    t += _gen(res, [x, f"{res}_ss", g], [_t([S, D], "bf16"), _t([S], "f32"), _t([D], "f32")],
              "bf16", [S, D], [idd, row, col, idd], ["parallel", "parallel"],
              ["%a: bf16", "%s: f32", "%g: f32", "%o: bf16"],
              [f"%d = arith.constant {float(D)!r} : f32", f"%eps = arith.constant {eps!r} : f32",
               "%one = arith.constant 1.0 : f32", "%e = arith.extf %a : bf16 to f32",
               "%ms = arith.divf %s, %d : f32", "%v = arith.addf %ms, %eps : f32",
               "%r = math.sqrt %v : f32", "%inv = arith.divf %one, %r : f32",
               "%t = arith.mulf %e, %inv : f32", "%u = arith.mulf %t, %g : f32",
               "%b = arith.truncf %u : f32 to bf16"], "%b")
    return t


def _mm(res, a, w, M, K, N, ea="bf16"):
    t = _fill(f"{res}_f", [M, N], "f32", "%zf")
    return t + (f"  {res} = linalg.matmul ins({a}, {w} : {_t([M, K], ea)}, {_t([K, N], 'bf16')}) "
                f"outs({res}_f : {_t([M, N], 'f32')}) -> {_t([M, N], 'f32')}\n")


def _residual(res, r, acc, S, N):
    idd = _amap(2, "d0, d1")
    return _gen(res, [r, acc], [_t([S, N], "bf16"), _t([S, N], "f32")], "bf16", [S, N],
                [idd, idd, idd], ["parallel", "parallel"], ["%r: bf16", "%a: f32", "%o: bf16"],
                ["%e = arith.extf %r : bf16 to f32", "%s = arith.addf %e, %a : f32",
                 "%t = arith.truncf %s : f32 to bf16"], "%t")


def _trunc(res, a, shape):
    idd = _amap(len(shape), ", ".join(f"d{i}" for i in range(len(shape))))
    return _gen(res, [a], [_t(shape, "f32")], "bf16", shape, [idd, idd],
                ["parallel"] * len(shape), ["%a: f32", "%o: bf16"],
                ["%t = arith.truncf %a : f32 to bf16"], "%t")


def _rope(res, acc, S, D, H, dh=64):
    """res (bf16, [S, D]) = RoPE of the f32 accumulator on interleaved pairs:
    (x0, x1) -> (x0 c - x1 s, x0 s + x1 c), over the [S, H, dh / 2, 2] view."""
    v4 = [S, H, dh // 2, 2]
    t = (f"  {res}_4 = tensor.expand_shape {acc} [[0], [1, 2, 3]] output_shape [{S}, {H}, {dh // 2}, 2] "
         f": {_t([S, D], 'f32')} into {_t(v4, 'f32')}\n")
    t += _gen(f"{res}_r", [f"{res}_4", f"{res}_4", "%cos", "%sin"],
              [_t(v4, "f32"), _t(v4, "f32"), _t([S, dh // 2], "f32"), _t([S, dh // 2], "f32")],
              "bf16", v4,
              [_amap(4, "d0, d1, d2, 0"), _amap(4, "d0, d1, d2, 1"), _amap(4, "d0, d2"),
               _amap(4, "d0, d2"), _amap(4, "d0, d1, d2, d3")], ["parallel"] * 4,
              ["%x0: f32", "%x1: f32", "%c: f32", "%s: f32", "%o: bf16"],
              ["%a = arith.mulf %x0, %c : f32", "%b = arith.mulf %x1, %s : f32",
               "%e = arith.mulf %x0, %s : f32", "%f = arith.mulf %x1, %c : f32",
               "%ev = arith.subf %a, %b : f32", "%od = arith.addf %e, %f : f32",
               "%j = linalg.index 3 : index", "%c0 = arith.constant 0 : index",
               "%is0 = arith.cmpi eq, %j, %c0 : index", "%v = arith.select %is0, %ev, %od : f32",
               "%t = arith.truncf %v : f32 to bf16"], "%t")
    t += (f"  {res} = tensor.collapse_shape {res}_r [[0], [1, 2, 3]] : {_t(v4, 'bf16')} into "
          f"{_t([S, D], 'bf16')}\n")
    return t


def _heads(res, v, S, H, perm, dh=64):
    """[S, D] -> [S, H, dh] -> transposed by `perm` (bf16)."""
    s3 = [S, H, dh]
    out = [s3[p] for p in perm]
    return (f"  {res}_3 = tensor.expand_shape {v} [[0], [1, 2]] output_shape [{S}, {H}, {dh}] : "
            f"{_t([S, H * dh], 'bf16')} into {_t(s3, 'bf16')}\n"
            f"  {res}_e = tensor.empty() : {_t(out, 'bf16')}\n"
            f"  {res} = linalg.transpose ins({res}_3 : {_t(s3, 'bf16')}) outs({res}_e : "
            f"{_t(out, 'bf16')}) permutation = [{', '.join(map(str, perm))}]\n")


def _attention(res, Q, K, V, S, H, scale, dh=64):
    """Causal softmax attention per head, in the oracle's order: S = Q K^T,
    scaled, keys after the query set to -inf, softmax (max, exp, sum,
    divide) in f32, O = P V, A = bf16(O) as [S, D]."""
    D = H * dh
    id3, row3 = _amap(3, "d0, d1, d2"), _amap(3, "d0, d1")
    t = _heads(f"{res}_q", Q, S, H, [1, 0, 2], dh) + _heads(f"{res}_k", K, S, H, [1, 2, 0], dh) + \
        _heads(f"{res}_v", V, S, H, [1, 0, 2], dh)
    t += _fill(f"{res}_s0", [H, S, S], "f32", "%zf")
    t += (f"  {res}_s = linalg.batch_matmul ins({res}_q, {res}_k : {_t([H, S, dh], 'bf16')}, "
          f"{_t([H, dh, S], 'bf16')}) outs({res}_s0 : {_t([H, S, S], 'f32')}) -> "
          f"{_t([H, S, S], 'f32')}\n")
    t += _gen(f"{res}_sm", [f"{res}_s"], [_t([H, S, S], "f32")], "f32", [H, S, S], [id3, id3],
              ["parallel"] * 3, ["%a: f32", "%o: f32"],
              [f"%sc = arith.constant {scale!r} : f32", "%v = arith.mulf %a, %sc : f32",
               "%i = linalg.index 1 : index", "%j = linalg.index 2 : index",
               "%gt = arith.cmpi ugt, %j, %i : index", "%ninf = arith.constant 0xFF800000 : f32",
               "%r = arith.select %gt, %ninf, %v : f32"], "%r")
    t += _fill(f"{res}_m0", [H, S], "f32", "%ninf")
    t += _gen(f"{res}_m", [f"{res}_sm"], [_t([H, S, S], "f32")], "f32", [H, S], [id3, row3],
              ["parallel", "parallel", "reduction"], ["%a: f32", "%acc: f32"],
              ["%m = arith.maximumf %acc, %a : f32"], "%m", init=f"{res}_m0")
    t += _gen(f"{res}_x", [f"{res}_sm", f"{res}_m"], [_t([H, S, S], "f32"), _t([H, S], "f32")],
              "f32", [H, S, S], [id3, row3, id3], ["parallel"] * 3, ["%a: f32", "%m: f32", "%o: f32"],
              ["%d = arith.subf %a, %m : f32", "%e = math.exp %d : f32"], "%e")
    t += _fill(f"{res}_l0", [H, S], "f32", "%zf")
    t += _gen(f"{res}_l", [f"{res}_x"], [_t([H, S, S], "f32")], "f32", [H, S], [id3, row3],
              ["parallel", "parallel", "reduction"], ["%a: f32", "%acc: f32"],
              ["%s = arith.addf %acc, %a : f32"], "%s", init=f"{res}_l0")
    t += _gen(f"{res}_p", [f"{res}_x", f"{res}_l"], [_t([H, S, S], "f32"), _t([H, S], "f32")],
              "f32", [H, S, S], [id3, row3, id3], ["parallel"] * 3, ["%a: f32", "%l: f32", "%o: f32"],
              ["%r = arith.divf %a, %l : f32"], "%r")
    t += _fill(f"{res}_o0", [H, S, dh], "f32", "%zf")
    t += (f"  {res}_o = linalg.batch_matmul ins({res}_p, {res}_v : {_t([H, S, S], 'f32')}, "
          f"{_t([H, S, dh], 'bf16')}) outs({res}_o0 : {_t([H, S, dh], 'f32')}) -> "
          f"{_t([H, S, dh], 'f32')}\n")
    t += (f"  {res}_ot_e = tensor.empty() : {_t([S, H, dh], 'f32')}\n"
          f"  {res}_ot = linalg.transpose ins({res}_o : {_t([H, S, dh], 'f32')}) outs({res}_ot_e : "
          f"{_t([S, H, dh], 'f32')}) permutation = [1, 0, 2]\n"
          f"  {res}_o2 = tensor.collapse_shape {res}_ot [[0], [1, 2]] : {_t([S, H, dh], 'f32')} "
          f"into {_t([S, D], 'f32')}\n")
    return t + _trunc(res, f"{res}_o2", [S, D])


def llama_layer(S, D, H, F, eps=1e-05, dh=None):
    """C5, one Llama decoder layer in bf16 storage (the oracle's semantics):
    RMSNorm -> Q, K, V projections (RoPE on Q and K) -> causal softmax
    attention -> O projection + x -> RMSNorm -> gate / up projections, SiLU
    gating -> down projection + h.  The reference's test/llama_attention.mlir
    replaces softmax by ReLU and has no norm, RoPE or gating; this is the real
    layer, written with the ops the reference's passes read."""
    dh = dh or D // H
    scale = 1.0 / math.sqrt(dh)
    sig = (f"%x: {_t([S, D], 'bf16')}, %g1: {_t([D], 'f32')}, %wq: {_t([D, D], 'bf16')}, "
           f"%wk: {_t([D, D], 'bf16')}, %wv: {_t([D, D], 'bf16')}, %wo: {_t([D, D], 'bf16')}, "
           f"%g2: {_t([D], 'f32')}, %wg: {_t([D, F], 'bf16')}, %wu: {_t([D, F], 'bf16')}, "
           f"%wd: {_t([F, D], 'bf16')}, %cos: {_t([S, dh // 2], 'f32')}, "
           f"%sin: {_t([S, dh // 2], 'f32')}")
    t = (f"func.func @llama_layer({sig}) -> {_t([S, D], 'bf16')} {{\n"
         f"  %zf = arith.constant 0.0 : f32\n  %ninf = arith.constant 0xFF800000 : f32\n")
    t += _rmsnorm("%xn", "%x", "%g1", S, D, eps)
    t += _mm("%qa", "%xn", "%wq", S, D, D) + _mm("%ka", "%xn", "%wk", S, D, D) + \
        _mm("%va", "%xn", "%wv", S, D, D)
    t += _rope("%Q", "%qa", S, D, H, dh) + _rope("%K", "%ka", S, D, H, dh) + \
        _trunc("%V", "%va", [S, D])
    t += _attention("%A", "%Q", "%K", "%V", S, H, scale, dh)
    t += _mm("%oa", "%A", "%wo", S, D, D) + _residual("%h", "%x", "%oa", S, D)
    t += _rmsnorm("%hn", "%h", "%g2", S, D, eps)
    t += _mm("%ga", "%hn", "%wg", S, D, F) + _mm("%ua", "%hn", "%wu", S, D, F)
    idd = _amap(2, "d0, d1")
    t += _gen("%act", ["%ga", "%ua"], [_t([S, F], "f32"), _t([S, F], "f32")], "bf16", [S, F],
              [idd, idd, idd], ["parallel", "parallel"], ["%g: f32", "%u: f32", "%o: bf16"],
              ["%n = arith.negf %g : f32", "%e = math.exp %n : f32",
               "%one = arith.constant 1.0 : f32", "%den = arith.addf %one, %e : f32",
               "%s = arith.divf %g, %den : f32", "%m = arith.mulf %s, %u : f32",
               "%t = arith.truncf %m : f32 to bf16"], "%t")
    t += _mm("%da", "%act", "%wd", S, F, D) + _residual("%out", "%h", "%da", S, D)
    return t + f"  return %out : {_t([S, D], 'bf16')}\n}}\n"


def _nchw_conv(res, x, w, xs, ws, os_, elem):
    return (f"  {res}_i = tensor.empty() : {_t(os_, elem)}\n"
            f"  {res}_f = linalg.fill ins(%cst : {elem}) outs({res}_i : {_t(os_, elem)}) -> "
            f"{_t(os_, elem)}\n"
            f"  {res} = linalg.conv_2d_nchw_fchw {{dilations = dense<1> : tensor<2xi64>, "
            f"strides = dense<1> : tensor<2xi64>}}\n"
            f"    ins({x}, {w} : {_t(xs, elem)}, {_t(ws, elem)}) outs({res}_f : {_t(os_, elem)}) "
            f"-> {_t(os_, elem)}\n")


def _nchw_eltwise(res, ins, shape, elem, body, yielded):
    ids = ", ".join(f"d{i}" for i in range(4))
    full = f"affine_map<({ids}) -> ({ids})>"
    args = ", ".join([f"%a{i}: {elem}" for i in range(len(ins))] + [f"%out: {elem}"])
    its = ", ".join(['"parallel"'] * 4)
    return (f"  {res}_e = tensor.empty() : {_t(shape, elem)}\n"
            f"  {res} = linalg.generic {{indexing_maps = [{', '.join([full] * (len(ins) + 1))}],\n"
            f"    iterator_types = [{its}]}} "
            f"ins({', '.join(ins)} : {', '.join([_t(shape, elem)] * len(ins))}) "
            f"outs({res}_e : {_t(shape, elem)}) {{\n  ^bb0({args}):\n" +
            "".join(f"    {b}\n" for b in body) + f"    linalg.yield {yielded} : {elem}\n"
            f"  }} -> {_t(shape, elem)}\n")


def model_zoo_bottleneck(N, C, M, H, W, final_relu, elem="f16", name="bottleneck"):
    """A stride-1 residual block in the form of the reference's model-zoo
    texts (tools/gen_model_mlir.py's output): NCHW, f16, a 1x1 conv C -> M,
    ReLU, a zero pad of 1, a 3x3 conv M -> M written as a dense conv (the
    generator emits no depthwise convolutions), ReLU, a 1x1 conv M -> C, a
    generic adding the block's input and, for a ResNet bottleneck, a ReLU
    generic after it.  test/models/resnet50.mlir:194-267 (C = 256, M = 64,
    final ReLU) and test/models/mobilenetv2.mlir:166-226 (the inverted
    residual block: C = 24, M = 144, none) have this form; this builder
    writes it with the same ops, shapes, maps and bodies."""
    xs, es = [N, C, H, W], [N, M, H, W]
    ps = [N, M, H + 2, W + 2]
    t = (f"func.func @{name}(%x: {_t(xs, elem)}, %w1: {_t([M, C, 1, 1], elem)}, "
         f"%w2: {_t([M, M, 3, 3], elem)}, %w3: {_t([C, M, 1, 1], elem)}) -> "
         f"{_t(xs, elem)} {{\n  %cst = arith.constant 0.0 : {elem}\n")
    relu = [f"%z = arith.constant 0.0 : {elem}", f"%m = arith.maximumf %a0, %z : {elem}"]
    t += _nchw_conv("%c1", "%x", "%w1", xs, [M, C, 1, 1], es, elem)
    t += _nchw_eltwise("%r1", ["%c1"], es, elem, relu, "%m")
    t += (f"  %p = tensor.pad %r1 low[0, 0, 1, 1] high[0, 0, 1, 1] {{\n"
          f"  ^bb0(%i0: index, %i1: index, %i2: index, %i3: index):\n"
          f"    tensor.yield %cst : {elem}\n  }} : {_t(es, elem)} to {_t(ps, elem)}\n")
    t += _nchw_conv("%c2", "%p", "%w2", ps, [M, M, 3, 3], es, elem)
    t += _nchw_eltwise("%r2", ["%c2"], es, elem, relu, "%m")
    t += _nchw_conv("%c3", "%r2", "%w3", es, [C, M, 1, 1], xs, elem)
    t += _nchw_eltwise("%s", ["%c3", "%x"], xs, elem, [f"%s = arith.addf %a0, %a1 : {elem}"], "%s")
    y = "%s"
    if final_relu:
        t += _nchw_eltwise("%y", ["%s"], xs, elem, relu, "%m")
        y = "%y"
    return t + f"  return {y} : {_t(xs, elem)}\n}}\n"


def _nchw_pad(res, x, shape, p, elem):
    ps = [shape[0], shape[1], shape[2] + 2 * p, shape[3] + 2 * p]
    return (f"  {res} = tensor.pad {x} low[0, 0, {p}, {p}] high[0, 0, {p}, {p}] {{\n"
            f"  ^bb0(%i0: index, %i1: index, %i2: index, %i3: index):\n"
            f"    tensor.yield %cst : {elem}\n  }} : {_t(shape, elem)} to {_t(ps, elem)}\n")


def nchw_conv_relu(N, C, F, H, W, elem="f16"):
    """test/conv2d_relu.mlir's form: a zero pad of 1 in H and W, then fill ->
    conv_2d_nchw_fchw 3x3 -> ReLU generic (`arith.maximumf` with 0)."""
    xs, os_, ps = [N, C, H, W], [N, F, H, W], [N, C, H + 2, W + 2]
    relu = [f"%z = arith.constant 0.0 : {elem}", f"%m = arith.maximumf %a0, %z : {elem}"]
    return (f"func.func @conv2d_relu(%input: {_t(xs, elem)}, %filter: {_t([F, C, 3, 3], elem)}) "
            f"-> {_t(os_, elem)} {{\n  %cst = arith.constant 0.0 : {elem}\n" +
            _nchw_pad("%p", "%input", xs, 1, elem) +
            _nchw_conv("%c", "%p", "%filter", ps, [F, C, 3, 3], os_, elem) +
            _nchw_eltwise("%r", ["%c"], os_, elem, relu, "%m") +
            f"  return %r : {_t(os_, elem)}\n}}\n")


def nchw_conv_bias_act(N, C, F, H, W, act="relu", elem="f32"):
    """A zero pad of 1 in H and W, then fill -> conv_2d_nchw_fchw 3x3 ->
    generic(bias along the output channels, activation)."""
    xs, os_, ps = [N, C, H, W], [N, F, H, W], [N, C, H + 2, W + 2]
    return (f"func.func @conv2d_bias_act(%input: {_t(xs, elem)}, %filter: "
            f"{_t([F, C, 3, 3], elem)}, %bias: {_t([F], elem)}) -> {_t(os_, elem)} {{\n"
            f"  %cst = arith.constant 0.0 : {elem}\n" +
            _nchw_pad("%p", "%input", xs, 1, elem) +
            _nchw_conv("%c", "%p", "%filter", ps, [F, C, 3, 3], os_, elem) +
            _epilogue("%r", "%c", "%bias", os_, elem, act, bias_dim=1) +
            f"  return %r : {_t(os_, elem)}\n}}\n")


def nchw_resnet_block(N, C, H, W, elem="f16"):
    """test/resnet_block.mlir's form: pad -> 3x3 conv -> ReLU -> pad -> 3x3
    conv -> generic adding the block's input (no ReLU after it)."""
    xs, ps = [N, C, H, W], [N, C, H + 2, W + 2]
    ws = [C, C, 3, 3]
    relu = [f"%z = arith.constant 0.0 : {elem}", f"%m = arith.maximumf %a0, %z : {elem}"]
    return (f"func.func @resnet_block(%input: {_t(xs, elem)}, %w1: {_t(ws, elem)}, "
            f"%w2: {_t(ws, elem)}) -> {_t(xs, elem)} {{\n  %cst = arith.constant 0.0 : {elem}\n" +
            _nchw_pad("%p1", "%input", xs, 1, elem) +
            _nchw_conv("%c1", "%p1", "%w1", ps, ws, xs, elem) +
            _nchw_eltwise("%r1", ["%c1"], xs, elem, relu, "%m") +
            _nchw_pad("%p2", "%r1", xs, 1, elem) +
            _nchw_conv("%c2", "%p2", "%w2", ps, ws, xs, elem) +
            _nchw_eltwise("%s", ["%c2", "%input"], xs, elem,
                          [f"%s = arith.addf %a0, %a1 : {elem}"], "%s") +
            f"  return %s : {_t(xs, elem)}\n}}\n")


def model_zoo_irb(N, C, E, H, W, elem="f16"):
    """The inverted residual block of stride 1 in the model-zoo form
    (test/models/mobilenetv2.mlir:166-226): model_zoo_bottleneck with the
    expansion E as the middle width and no ReLU after the add."""
    return model_zoo_bottleneck(N, C, E, H, W, False, elem, name="irb")
