"""Frontends: a torch module, or the reference's NCHW model texts, as the NHWC
linalg the host lowering (npu_amd.lower) runs on the MI355X.

The reference reaches linalg two ways: tools/torch2npu.py exports a torch model
to ONNX and writes NCHW linalg from the ONNX graph (`_conv`, `_matmul`, `_relu`,
`_add`, :199-355; normalisation, pooling and reshapes passed through, :163-197),
and tools/gen_model_mlir.py writes the model-zoo texts (test/models/*.mlir)
directly, NCHW and f16.  The kernels here take channels last, so:

* ``from_torch(module, x)`` traces the module with torch.fx (no ONNX step) and
  writes NHWC linalg for what the entry points execute: ``nn.Conv2d`` (dense
  or depthwise, stride 1, symmetric zero padding), ``nn.BatchNorm2d`` after a
  conv folded into its filters and bias (inference form), ``nn.ReLU`` /
  ``nn.ReLU6`` / ``F.relu``, ``nn.Linear`` (its weight passed transposed, as
  ``linalg.matmul`` takes ``[K, N]``) and a residual ``+``.  Each conv or
  linear and the elementwise ops after it become one fill -> op -> generic
  chain, the generic holding the bias, the residual and the activation.  It
  returns the text and the argument tensors (channels last).  Anything else
  raises NotImplementedError naming the node.
* ``nchw_to_nhwc(func)`` rewrites a function in the model texts' form --
  ``conv_2d_nchw_fchw``, elementwise generics over NCHW tensors,
  ``tensor.pad`` -- into the NHWC form: activations [N,C,H,W] -> [N,H,W,C],
  filters [F,C,KH,KW] -> [F,KH,KW,C], the generics' iteration spaces and
  maps permuted the same way, the pads' low/high likewise.
* ``extract_block(func, inputs, output)`` is the ops computing ``output``
  from ``inputs`` (and the function's arguments), as a function of its own:
  one block of a model-zoo text, e.g. the inverted residual block at
  test/models/mobilenetv2.mlir:166-226.

* ``from_torch_int8(module, calib)`` quantizes a float ResNet bottleneck
  (1x1 conv, ReLU, 3x3 conv, ReLU, 1x1 conv, + input, ReLU; no conv biases)
  after training: filters per output channel, symmetric, to [-127, 127];
  activations with zero point 0, the block's input and output at scale
  1/127 (so the residual adds directly), the two inner activations at the
  scale that maps their 99.9th percentile on the calibration batch to 127;
  each requantization's multiplier and shift the fixed-point form of
  s_in * s_w[c] / s_out.  Returns the int8 NHWC linalg text the int8
  bottleneck's lowering runs and its argument arrays.

``emit(func)`` prints a parsed function back as text.
"""
from __future__ import annotations

from . import mlir

_NHWC = [0, 2, 3, 1]        # new dim i <- old (NCHW) dim _NHWC[i]
_NHWC_INV = [0, 3, 1, 2]    # old dim j -> new dim


# ------------------------------------------------------------------ printing
def _ty(t):
    return str(t)


def _map_text(rank, res):
    ids = ", ".join(f"d{i}" for i in range(rank))
    exprs = ", ".join(f"d{r}" if isinstance(r, int) else str(r) for r in res)
    return f"affine_map<({ids}) -> ({exprs})>"


def _body_text(op):
    lines = []
    for b in op.attrs.get("body", []):
        if b.name == "arith.constant":
            lines.append(f"    {b.result} = arith.constant {b.value} : {b.type}")
        elif b.name == "linalg.index":
            lines.append(f"    {b.result} = linalg.index {b.value} : {b.type}")
        elif b.name in ("arith.cmpi", "arith.cmpf"):
            lines.append(f"    {b.result} = {b.name} {b.value}, {', '.join(b.operands)} : {b.type}")
        else:
            lines.append(f"    {b.result} = {b.name} {', '.join(b.operands)} : {b.type}")
    return lines


def _op_text(op, types):
    r = op.results[0] if op.results else None
    if op.name == "arith.constant":
        return f"  {r} = arith.constant {op.attrs['value']} : {_ty(op.result_types[0])}"
    if op.name == "tensor.empty":
        return f"  {r} = tensor.empty() : {_ty(types[r])}"
    if op.name == "tensor.pad":
        lo = ", ".join(map(str, op.attrs["low"]))
        hi = ", ".join(map(str, op.attrs["high"]))
        src = op.operands[0]
        n = len(op.attrs["low"])
        bb = ", ".join(f"%i{k}: index" for k in range(n))
        return (f"  {r} = tensor.pad {src} low[{lo}] high[{hi}] {{\n  ^bb0({bb}):\n"
                f"    tensor.yield {op.attrs['yield']} : {types[r].elem}\n"
                f"  }} : {_ty(types[src])} to {_ty(types[r])}")
    if op.name == "func.return":
        return f"  return {', '.join(op.operands)} : {', '.join(_ty(types[v]) for v in op.operands)}"
    if op.name.startswith("linalg."):
        ins_t = ", ".join(_ty(types[v]) if v in types else types.get(v, "f32") for v in op.ins)
        outs_t = ", ".join(_ty(types[v]) for v in op.outs)
        res_t = _ty(types[r])
        if op.name == "linalg.fill":
            return (f"  {r} = linalg.fill ins({op.ins[0]} : {types[op.ins[0]].elem}) "
                    f"outs({op.outs[0]} : {outs_t}) -> {res_t}")
        if op.name == "linalg.generic":
            rank = len(op.iterators)
            maps = ", ".join(_map_text(rank, m) for m in op.attrs["maps"])
            it = ", ".join(f'"{x}"' for x in op.iterators)
            args = ", ".join(f"{a}: {t}" for a, t in zip(
                op.attrs["block_args"], [types[v].elem for v in op.ins + op.outs]))
            body = "\n".join(_body_text(op))
            y = op.attrs["yield"][0]
            return (f"  {r} = linalg.generic {{indexing_maps = [{maps}],\n"
                    f"    iterator_types = [{it}]}} ins({', '.join(op.ins)} : {ins_t}) "
                    f"outs({', '.join(op.outs)} : {outs_t}) {{\n  ^bb0({args}):\n{body}\n"
                    f"    linalg.yield {y} : {types[r].elem}\n  }} -> {res_t}")
        attrs = ""
        if "conv" in op.name:
            st = op.attrs.get("strides", [1, 1])
            attrs = (" {dilations = dense<1> : tensor<2xi64>, "
                     f"strides = dense<[{st[0]}, {st[1]}]> : tensor<2xi64>}}")
        return (f"  {r} = {op.name}{attrs} ins({', '.join(op.ins)} : {ins_t}) "
                f"outs({', '.join(op.outs)} : {outs_t}) -> {res_t}")
    raise NotImplementedError(f"{r}: {op.name} has no printer here")


def emit(func: mlir.MFunc) -> str:
    """The function as MLIR text (the op forms the lowering reads)."""
    sig = ", ".join(f"{a}: {_ty(t)}" for a, t in func.args)
    rt = ", ".join(_ty(t) for t in func.result_types)
    lines = [f"func.func @{func.name}({sig}) -> {rt} {{"]
    types = dict(func.types)
    for op in func.ops:
        lines.append(_op_text(op, types))
    lines.append("}")
    return "\n".join(lines) + "\n"


# ------------------------------------------------------------------ blocks
def extract_block(func: mlir.MFunc, inputs, output, name=None) -> mlir.MFunc:
    """The ops computing `output` from `inputs` and the function's arguments,
    as a function whose arguments are `inputs`, then the function arguments
    the block reads (in the function's order), returning `output`."""
    inputs = list(inputs)
    prod = {r: op for op in func.ops for r in op.results}
    need, stack = set(), [output]
    while stack:
        v = stack.pop()
        if v in need or v in inputs:
            continue
        op = prod.get(v)
        if op is None:
            continue  # a function argument
        need.add(v)
        operands = op.all_operands + ([op.attrs["yield"]] if op.name == "tensor.pad" else [])
        stack.extend(o for o in operands if o)
    ops = [op for op in func.ops if op.results and op.results[0] in need]
    used = {o for op in ops for o in op.all_operands}
    used |= {op.attrs["yield"] for op in ops if op.name == "tensor.pad"}
    args = [(v, func.types[v]) for v in inputs]
    args += [(a, t) for a, t in func.args if a in used and a not in inputs]
    ret = mlir.MOp("func.return", [], [], operands=[output])
    return mlir.MFunc(name or f"{func.name}_block", args, [func.types[output]], ops + [ret],
                      {**{a: t for a, t in args}, **{r: func.types[r] for op in ops for r in op.results}},
                      func.target)


# ------------------------------------------------------------------ NCHW -> NHWC
def _permute(shape, perm):
    return [shape[p] for p in perm]


def nchw_to_nhwc(func: mlir.MFunc) -> mlir.MFunc:
    """The function with its NCHW convolutions and the rank-4 values around
    them in channels-last form (module docstring)."""
    filters = set()
    for op in func.ops:
        if op.name == "linalg.conv_2d_nchw_fchw":
            filters.add(op.ins[1])
        elif op.name.startswith("linalg.conv") or op.name.startswith("linalg.depthwise") or \
                op.name.startswith("linalg.pooling"):
            raise NotImplementedError(f"{op.results[0]}: {op.name} (only conv_2d_nchw_fchw is "
                                      "rewritten)")
    types = {}
    for v, t in func.types.items():
        if t.shaped and len(t.shape) == 4:
            perm = [0, 2, 3, 1]
            types[v] = mlir.TType(_permute(t.shape, perm), t.elem)
        else:
            types[v] = t
    # filters [F,C,KH,KW] -> [F,KH,KW,C]: the same permutation
    ops = []
    for op in func.ops:
        new = mlir.MOp(op.name, list(op.results), [types[r] for r in op.results], list(op.ins),
                       list(op.outs), list(op.operands), list(op.iterators), list(op.body_ops),
                       dict(op.attrs), op.text)
        if op.name == "linalg.conv_2d_nchw_fchw":
            new.name = "linalg.conv_2d_nhwc_fhwc"
        elif op.name == "tensor.pad":
            if len(op.attrs["low"]) == 4:
                new.attrs["low"] = _permute(op.attrs["low"], _NHWC)
                new.attrs["high"] = _permute(op.attrs["high"], _NHWC)
        elif op.name == "linalg.generic":
            rank = len(op.iterators)
            operands = op.ins + op.outs
            ranks = [len(func.types[v].shape) for v in operands]
            if rank == 4:
                new.iterators = _permute(op.iterators, _NHWC)
                maps = []
                for m, vr in zip(op.attrs["maps"], ranks):
                    if any(not isinstance(e, int) for e in m):
                        raise NotImplementedError(f"{op.results[0]}: generic map with constants")
                    m2 = [_NHWC_INV[e] for e in m]          # renumber the loop dims
                    if vr == 4:
                        m2 = _permute(m2, _NHWC)            # the operand's own dims
                    maps.append(m2)
                new.attrs["maps"] = maps
            elif any(r == 4 for r in ranks):
                raise NotImplementedError(f"{op.results[0]}: a generic of rank {rank} over a "
                                          "rank-4 tensor")
        elif op.name.startswith("linalg.") and op.name not in ("linalg.fill",):
            if any(len(func.types[v].shape) == 4 for v in op.ins + op.outs if v in func.types
                   and func.types[v].shaped):
                raise NotImplementedError(f"{op.results[0]}: {op.name} over a rank-4 tensor")
        ops.append(new)
    args = [(a, types[a]) for a, _ in func.args]
    rts = [types[v] for v in (ops[-1].operands if ops and ops[-1].name == "func.return" else [])]
    return mlir.MFunc(func.name, args, rts or func.result_types, ops, types, func.target)


# ------------------------------------------------------------------ torch
_ELEM = {"torch.float32": "f32", "torch.bfloat16": "bf16"}


class _Writer:
    def __init__(self, elem):
        self.elem = elem
        self.lines = []
        self.args = []        # (name, shape, elem, tensor)
        self.n = 0

    def fresh(self, stem):
        self.n += 1
        return f"%{stem}{self.n}"

    def arg(self, stem, tensor, elem=None):
        name = f"%{stem}{len(self.args)}"
        self.args.append((name, list(tensor.shape), elem or self.elem, tensor))
        return name


def from_torch(module, x, elem="f32", name="model"):
    """(text, {argument name: tensor}) of `module` applied to the NCHW input
    `x`, as NHWC linalg (module docstring).  The tensors are the argument
    values in channels-last layout (the input, folded filters, transposed
    linear weights, biases), on the CPU, float32 (or bfloat16 for elem="bf16";
    biases stay float32)."""
    import operator

    import torch
    import torch.fx
    from torch.fx.passes.shape_prop import ShapeProp

    from .blocks import _conv, _epilogue, _pad, _t

    module = module.eval()
    gm = torch.fx.symbolic_trace(module)
    ShapeProp(gm).propagate(x)
    mods = dict(gm.named_modules())
    tdt = torch.float32 if elem == "f32" else torch.bfloat16
    w = _Writer(elem)
    vals = {}      # fx node -> (ssa name, shape in the text's layout)

    def users(n):
        return list(n.users)

    def single_user(n):
        u = users(n)
        return u[0] if len(u) == 1 else None

    def kind(n):
        if n.op == "call_module":
            return type(mods[n.target]).__name__
        if n.op == "call_function":
            if n.target in (operator.add, torch.add):
                return "add"
            if n.target in (torch.relu, torch.nn.functional.relu):
                return "ReLU"
            if n.target is torch.nn.functional.relu6:
                return "ReLU6"
            return getattr(n.target, "__name__", str(n.target))
        if n.op == "call_method" and n.target == "relu":
            return "ReLU"
        return n.op

    consumed = set()

    def epilogue_chain(n):
        """(residual node, act, last node) of the elementwise ops after `n`."""
        res, act, last = None, "none", n
        u = single_user(last)
        if u is not None and kind(u) == "add":
            if u.kwargs:
                # torch.add(y, x, alpha=a) scales x: not a plain residual add
                raise NotImplementedError(f"{u.name}: add with {sorted(u.kwargs)} "
                                          "(only a plain residual add is lowered)")
            other = [a for a in u.args if a is not last]
            if len(other) != 1 or len(u.args) != 2 or other[0] not in vals:
                raise NotImplementedError(f"{u.name}: an add that is not a residual of a "
                                          "computed value")
            res, last = other[0], u
            consumed.add(u)
            u = single_user(last)
        if u is not None and kind(u) in ("ReLU", "ReLU6"):
            act, last = kind(u).lower(), u
            consumed.add(u)
        return res, act, last

    for node in gm.graph.nodes:
        if node in consumed:
            continue
        k = kind(node)
        if node.op == "placeholder":
            t = x.permute(0, 2, 3, 1) if x.dim() == 4 else x
            vals[node] = (w.arg("x", t.contiguous().to(tdt)), list(t.shape))
        elif k == "Conv2d":
            m = mods[node.target]
            src, xs = vals[node.args[0]]
            if m.stride != (1, 1) or m.dilation != (1, 1) or m.padding_mode != "zeros" or \
                    not isinstance(m.padding, tuple) or m.padding[0] != m.padding[1] or \
                    m.kernel_size[0] != m.kernel_size[1]:
                raise NotImplementedError(f"{node.name}: conv with stride {m.stride}, padding "
                                          f"{m.padding}, dilation {m.dilation}")
            wt = m.weight.detach().double()
            bias = m.bias.detach().double() if m.bias is not None else None
            u = single_user(node)
            if u is not None and kind(u) == "BatchNorm2d":
                bn = mods[u.target]
                s = bn.weight.detach().double() / torch.sqrt(bn.running_var.double() + bn.eps)
                wt = wt * s.view(-1, 1, 1, 1)
                bias = (bias if bias is not None else torch.zeros_like(s)) - bn.running_mean.double()
                bias = bias * s + bn.bias.detach().double()
                consumed.add(u)
                last0 = u
            else:
                last0 = node
            res, act, last = epilogue_chain(last0)
            p, K = m.padding[0], m.kernel_size[0]
            N, H, W_, C = xs
            F = m.out_channels
            os_ = [N, H + 2 * p - K + 1, W_ + 2 * p - K + 1, F]
            if p:
                pn = w.fresh("pad")
                text, xs = _pad(pn, src, xs, p, elem)
                w.lines.append(text)
                src = pn
            cn = w.fresh("conv")
            if m.groups == 1:
                wn = w.arg("w", wt.permute(0, 2, 3, 1).contiguous().to(tdt))
                w.lines.append(_conv(cn, src, wn, xs, [F, K, K, C], os_, elem))
            elif m.groups == C == F:
                wn = w.arg("w", wt[:, 0].permute(1, 2, 0).contiguous().to(tdt))
                w.lines.append(_conv(cn, src, wn, xs, [K, K, C], os_, elem,
                                     name="linalg.depthwise_conv_2d_nhwc_hwc"))
            else:
                raise NotImplementedError(f"{node.name}: grouped conv, groups {m.groups}")
            # the bias (or the folded batch norm's) in the text's element type:
            # a bf16 text holds it rounded to bf16, which the lowering widens
            # exactly to the f32 bias the entry point adds
            bn_ = w.arg("b", bias.to(tdt)) if bias is not None else None
            out = w.fresh("y")
            if bn_ is not None or res is not None or act != "none":
                w.lines.append(_epilogue(out, cn, bn_, os_, elem, act,
                                         residual=vals[res][0] if res is not None else None))
            else:
                out = cn
            vals[last] = (out, os_)
        elif k == "Linear":
            m = mods[node.target]
            src, xs = vals[node.args[0]]
            if len(xs) != 2:
                raise NotImplementedError(f"{node.name}: linear over a rank-{len(xs)} tensor")
            wn = w.arg("w", m.weight.detach().t().contiguous().to(tdt))
            bn_ = w.arg("b", m.bias.detach().to(tdt)) if m.bias is not None else None
            res, act, last = epilogue_chain(node)
            M, Kd = xs
            N_ = m.out_features
            init, fill, mm = w.fresh("init"), w.fresh("fill"), w.fresh("mm")
            w.lines.append(f"  {init} = tensor.empty() : {_t([M, N_], elem)}\n"
                           f"  {fill} = linalg.fill ins(%cst : {elem}) outs({init} : "
                           f"{_t([M, N_], elem)}) -> {_t([M, N_], elem)}\n"
                           f"  {mm} = linalg.matmul ins({src}, {wn} : {_t([M, Kd], elem)}, "
                           f"{_t([Kd, N_], elem)}) outs({fill} : {_t([M, N_], elem)}) -> "
                           f"{_t([M, N_], elem)}\n")
            out = w.fresh("y")
            if bn_ is not None or res is not None or act != "none":
                w.lines.append(_epilogue(out, mm, bn_, [M, N_], elem, act,
                                         residual=vals[res][0] if res is not None else None))
            else:
                out = mm
            vals[last] = (out, [M, N_])
        elif node.op == "output":
            ret = node.args[0]
            if not isinstance(ret, torch.fx.Node) or ret not in vals:
                raise NotImplementedError(f"output {ret}: not a value this frontend computed")
            rname, rshape = vals[ret]
            sig = ", ".join(f"{a}: {_t(s, e)}" for a, s, e, _ in w.args)
            text = (f"func.func @{name}({sig}) -> {_t(rshape, elem)} {{\n"
                    f"  %cst = arith.constant 0.0 : {elem}\n" + "".join(w.lines) +
                    f"  return {rname} : {_t(rshape, elem)}\n}}\n")
            return text, {a.lstrip("%"): t for a, _, _, t in w.args}
        else:
            raise NotImplementedError(f"{node.name}: {k} (the frontend writes conv, batch norm "
                                      "after a conv, linear, ReLU / ReLU6 and residual adds)")
    raise NotImplementedError("the module has no output")


def from_torch_int8(module, calib, name="qbottleneck"):
    """(text, {argument: numpy array}) of a float ResNet bottleneck quantized
    after training (module docstring).  `module` has the structure conv1
    (1x1, C -> M1), ReLU, conv2 (3x3, pad 1), ReLU, conv3 (1x1, M1 -> C), a
    residual add of the block input and a ReLU, with a batch norm after each
    conv allowed when it only scales (zero mean and shift): the int8 kernel
    adds no bias.  `calib` is an NCHW float batch with values in [0, 1]."""
    import operator

    import numpy as np
    import torch
    import torch.fx

    from . import blocks
    from .configs import _quantize_per_channel, quant_multiplier, requant_np

    module = module.eval()
    gm = torch.fx.symbolic_trace(module)
    mods = dict(gm.named_modules())
    convs, seq = [], []
    for n in gm.graph.nodes:
        if n.op == "call_module":
            m = mods[n.target]
            k = type(m).__name__
            if k == "Conv2d":
                if m.bias is not None and bool(torch.any(m.bias != 0)):
                    raise NotImplementedError(f"{n.name}: conv bias (the int8 kernel adds none)")
                if m.stride != (1, 1) or m.groups != 1 or m.dilation != (1, 1):
                    raise NotImplementedError(f"{n.name}: stride / groups / dilation")
                convs.append([m.weight.detach().double(), m.padding[0]])
                seq.append("conv")
            elif k == "BatchNorm2d":
                if not convs or seq[-1] != "conv":
                    raise NotImplementedError(f"{n.name}: batch norm not after a conv")
                sh = m.bias.detach().double() - m.running_mean.double() * m.weight.detach().double() \
                    / torch.sqrt(m.running_var.double() + m.eps)
                if bool(torch.any(sh.abs() > 1e-12)):
                    raise NotImplementedError(f"{n.name}: batch norm with a shift (a bias)")
                sc = m.weight.detach().double() / torch.sqrt(m.running_var.double() + m.eps)
                convs[-1][0] = convs[-1][0] * sc.view(-1, 1, 1, 1)
            elif k == "ReLU":
                seq.append("relu")
            else:
                raise NotImplementedError(f"{n.name}: {k}")
        elif n.op == "call_function":
            if n.target in (operator.add, torch.add):
                seq.append("add")
            elif n.target in (torch.relu, torch.nn.functional.relu):
                seq.append("relu")
            else:
                raise NotImplementedError(f"{n.name}: {n.target}")
        elif n.op == "call_method" and n.target == "relu":
            seq.append("relu")
    if seq != ["conv", "relu", "conv", "relu", "conv", "add", "relu"] or len(convs) != 3:
        raise NotImplementedError(f"not a bottleneck: {seq}")
    (w1f, p1), (w2f, p2), (w3f, p3) = convs
    M1, C = w1f.shape[0], w1f.shape[1]
    if (p1, p2, p3) != (0, 1, 0) or tuple(w1f.shape[2:]) != (1, 1) or \
            tuple(w2f.shape) != (M1, M1, 3, 3) or tuple(w3f.shape) != (C, M1, 1, 1):
        raise NotImplementedError("conv shapes are not 1x1 C->M1, 3x3 M1->M1, 1x1 M1->C")
    # weights per output channel; FHWC / [F, C] layouts of the int8 text
    w1, sw1 = _quantize_per_channel(w1f[:, :, 0, 0].numpy())
    w2, sw2 = _quantize_per_channel(w2f.permute(0, 2, 3, 1).numpy())
    w3, sw3 = _quantize_per_channel(w3f[:, :, 0, 0].numpy())
    xq = np.clip(np.rint(calib.permute(0, 2, 3, 1).double().numpy() * 127), 0, 127).astype(np.int8)
    N, H, W, _ = xq.shape
    sx = 1.0 / 127
    acc1 = xq.reshape(-1, C).astype(np.int64) @ w1.astype(np.int64).T
    sy1 = np.percentile(np.maximum(acc1 * (sx * sw1), 0), 99.9) / 127
    m1, s1 = quant_multiplier(sx * sw1 / sy1)
    y1 = np.clip(requant_np(acc1, m1, s1), 0, 127).reshape(N, H, W, M1)
    y1p = np.pad(y1, ((0, 0), (1, 1), (1, 1), (0, 0)))
    cols = np.concatenate([y1p[:, kh:kh + H, kw:kw + W] for kh in range(3) for kw in range(3)],
                          -1).reshape(-1, 9 * M1)
    acc2 = cols @ w2.reshape(M1, -1).astype(np.int64).T
    sy2 = np.percentile(np.maximum(acc2 * (sy1 * sw2), 0), 99.9) / 127
    m2, s2 = quant_multiplier(sy1 * sw2 / sy2)
    m3, s3 = quant_multiplier(sy2 * sw3 / sx)
    text = blocks.qbottleneck(N, H, W, C, M1).replace("@qbottleneck(", f"@{name}(")
    args = {"x": xq, "w1": w1.reshape(M1, 1, 1, C), "w2": w2, "w3": w3.reshape(C, 1, 1, M1),
            "m1": m1, "s1": s1, "m2": m2, "s2": s2, "m3": m3, "s3": s3}
    return text, args
