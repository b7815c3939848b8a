"""Host lowering: a linalg function -> calls of the fused-group entry points.

The reference lowers a fused group to a private function called from its tile
loop nest (`scf.for { extract_slice; func.call @fused_*; insert_slice }`,
lib/Transforms/OutlineFusedGroupsPass.cpp:306-316, SpatialTilingPass.cpp:138-166)
and runs the result with mlir-runner on the CPU (tools/harness/e2e_verify.py:232-251).
On the MI355X the whole loop nest of a group is one entry-point call
(include/npu_amd.h): `lower` runs the decision pipeline (npu_amd.pipeline), matches
each outlined group to the entry point that executes it, binds the group's values
to the function's arguments and to earlier calls' results, and returns a Program
that runs those calls on the GPU.  Matched:

* {fill, matmul, generic...}: bias add and ReLU / ReLU6 / none in the generic
  bodies -> fused_matmul_bias_act (f32);
* {fill, conv_2d_nhwc_fhwc, generic...}, its input optionally a tensor.pad of
  zeros symmetric in H and W -> fused_conv2d_nhwc_bias_act (f32 / bf16), the pad
  folded into the call;
* the inverted residual chain: {fill, 1x1 conv, ReLU6 generic} -> tensor.pad ->
  depthwise 3x3 -> ReLU6 generic -> 1x1 conv -> generic adding the chain's
  input (one group after the pad, or two: the fusion decision depends on the
  shapes) -> one fused_irb_f32 call (f32), the expanded tensor never leaving
  the chip.

Anything else -- an op no group covers, another dtype, a stride -- raises
NotImplementedError naming it: there is no fallback implementation.
"""
from __future__ import annotations

from dataclasses import dataclass, field

from . import mlir, pipeline


@dataclass
class Call:
    entry: str                 # entry point (include/npu_amd.h)
    functions: list            # outlined functions it executes
    args: list                 # SSA names in the entry point's operand order (None: absent)
    out: str                   # SSA name of the result
    params: dict = field(default_factory=dict)   # pad, act
    views: dict = field(default_factory=dict)    # SSA name -> shape the entry point takes


_TORCH_DTYPE = {"f32": "float32", "bf16": "bfloat16"}


def _act(body_ops):
    if "arith.minimumf" in body_ops:
        return "relu6"
    if "arith.maximumf" in body_ops:
        return "relu"
    return "none"


class _Fn:
    def __init__(self, func: mlir.MFunc):
        self.f = func
        self.producer = {}
        for i, op in enumerate(func.ops):
            for r in op.results:
                self.producer[r] = i

    def op(self, v):
        i = self.producer.get(v)
        return None if i is None else self.f.ops[i]

    def ty(self, v):
        return self.f.types[v]


def _epilogue(fn: _Fn, generics, src, shape):
    """Bias (a 1-D operand of the last dimension), residual (a same-shape
    operand) and activation of the generics that follow `src` in a group."""
    bias = residual = None
    act = "none"
    v = src
    for g in generics:
        if v not in g.ins:
            raise NotImplementedError(f"{g.results[0]}: epilogue not on the chain from {src}")
        for o in g.ins:
            if o == v:
                continue
            t = fn.ty(o)
            if t.shape == [shape[-1]] and bias is None:
                bias = o
            elif t.shape == list(shape) and residual is None:
                residual = o
            else:
                raise NotImplementedError(f"{g.results[0]}: operand {o} {t} in the epilogue")
        a = _act(g.body_ops)
        if a != "none":
            if act != "none":
                raise NotImplementedError(f"{g.results[0]}: a second activation")
            act = a
        v = g.results[0]
    return bias, residual, act, v


def _pad_of(fn: _Fn, v):
    """(source, pad) when v is a tensor.pad of zeros by p in H and W only."""
    op = fn.op(v)
    if op is None or op.name != "tensor.pad":
        return v, 0
    lo, hi = op.attrs.get("low", []), op.attrs.get("high", [])
    if len(lo) != 4 or lo != hi or lo[0] or lo[3] or lo[1] != lo[2]:
        raise NotImplementedError(f"{v}: pad low {lo} high {hi} (entry points pad H and W equally)")
    return op.operands[0], lo[1]


def _strided(op):
    return any(s != 1 for s in op.attrs.get("strides", [1, 1]))


def _elem(fn, v, allowed, what):
    e = fn.ty(v).elem
    if e not in allowed:
        raise NotImplementedError(f"{what}: element type {e} (entry point takes {'/'.join(allowed)})")
    return e


def lower(func: mlir.MFunc, target=None) -> "Program":
    """Matches func's outlined groups to entry points; see the module docstring."""
    fn = _Fn(func)
    rep = pipeline.run(func, target)
    groups = {g["name"]: [func.ops[i] for i in g["ops"]] for g in rep["functions"]}
    calls, covered, consumed = [], set(), set()
    kinds = lambda ops: [o.name for o in ops if o.name != "linalg.fill"]
    for name, ops in groups.items():
        if name in consumed:
            continue
        k = kinds(ops)
        gens = [o for o in ops if o.name == "linalg.generic"]
        if k[:1] == ["linalg.matmul"] and all(x == "linalg.generic" for x in k[1:]):
            mm = ops[[o.name for o in ops].index("linalg.matmul")]
            shape = fn.ty(mm.results[0]).shape
            bias, res, act, out = _epilogue(fn, gens, mm.results[0], shape)
            if res is not None:
                raise NotImplementedError(f"{name}: residual add after a matmul")
            _elem(fn, mm.ins[0], ("f32",), name)
            calls.append(Call("fused_matmul_bias_act", [name], [mm.ins[0], mm.ins[1], bias], out,
                              {"act": act}))
        elif k[:1] == ["linalg.conv_2d_nhwc_fhwc"] and all(x == "linalg.generic" for x in k[1:]):
            conv = ops[[o.name for o in ops].index("linalg.conv_2d_nhwc_fhwc")]
            if _strided(conv):
                raise NotImplementedError(f"{name}: strided convolution")
            shape = fn.ty(conv.results[0]).shape
            bias, res, act, out = _epilogue(fn, gens, conv.results[0], shape)
            x, pad = _pad_of(fn, conv.ins[0])
            # the expand group of an inverted residual chain: fold the chain
            chain = _irb_chain(fn, groups, name, conv, out, x, act, bias, res)
            if chain is not None:
                calls.append(chain)
                consumed.update(chain.functions)
                covered.update(r for f2 in chain.functions for o in groups[f2] for r in o.results)
                p = fn.op(chain.params["padded"])
                covered.update(p.results)
                continue
            if res is not None:
                raise NotImplementedError(f"{name}: residual add after a convolution")
            _elem(fn, x, ("f32", "bf16"), name)
            calls.append(Call("fused_conv2d_nhwc_bias_act", [name], [x, conv.ins[1], bias], out,
                              {"pad": pad, "act": act}))
            if pad:
                covered.add(conv.ins[0])
        else:
            raise NotImplementedError(f"{name}: no MI355X entry point runs ops {k}")
        covered.update(r for o in ops for r in o.results)
    # every computing op must be part of a call
    for op in func.ops:
        if op.name.startswith("linalg.") or op.name == "tensor.pad":
            if not op.results or op.results[0] not in covered:
                raise NotImplementedError(f"{op.results[0] if op.results else op.name}: "
                                          f"{op.name} is in no group an entry point runs")
    return Program(func, calls)


def _irb_chain(fn, groups, name, conv, e_out, x, act, bias, res):
    """The call running an inverted residual chain whose expand group is
    `name`, or None when the expand group is not followed by one."""
    if act != "relu6" or bias is not None or res is not None or x != conv.ins[0]:
        return None
    wshape = fn.ty(conv.ins[1]).shape
    if wshape[1:3] != [1, 1]:
        return None
    # the pad of e_out
    pads = [op for op in fn.f.ops if op.name == "tensor.pad" and op.operands[0] == e_out]
    if len(pads) != 1:
        return None
    ep = pads[0].results[0]
    _, p = _pad_of(fn, ep)
    if p != 1:
        return None
    # follow the values: depthwise(ep) -> ReLU6 -> 1x1 project -> + x, in one
    # group or two (the fusion decision depends on the shapes)
    group_of = {o.results[0]: n for n, ops in groups.items() for o in ops if o.results}

    def user(v, kind):
        us = [o for o in fn.f.ops if o.name == kind and v in o.ins]
        return us[0] if len(us) == 1 else None

    dw = user(ep, "linalg.depthwise_conv_2d_nhwc_hwc")
    g1 = dw and user(dw.results[0], "linalg.generic")
    if g1 is None:
        return None
    b1, r1, a1, d = _epilogue(fn, [g1], dw.results[0], fn.ty(dw.results[0]).shape)
    pr = user(d, "linalg.conv_2d_nhwc_fhwc")
    g2 = pr and user(pr.results[0], "linalg.generic")
    if g2 is None or (b1, r1, a1) != (None, None, "relu6") or _strided(dw) or _strided(pr):
        return None
    b2, r2, a2, y = _epilogue(fn, [g2], pr.results[0], fn.ty(pr.results[0]).shape)
    if (b2, a2) != (None, "none") or r2 != x:
        return None
    if fn.ty(pr.ins[1]).shape[1:3] != [1, 1] or fn.ty(dw.ins[1]).shape[:2] != [3, 3]:
        return None
    names = [name]
    for o in (dw, g1, pr, g2):
        n = group_of.get(o.results[0])
        if n is None:
            return None
        if n not in names:
            names.append(n)
    # the chain's groups hold only these ops (and fills)
    chain_ops = {id(o) for o in (dw, g1, pr, g2)}
    for n in names[1:]:
        if any(o.name != "linalg.fill" and id(o) not in chain_ops for o in groups[n]):
            return None
    _elem(fn, x, ("f32",), names[-1])
    E, C = wshape[0], wshape[3]
    return Call("fused_irb_f32", names, [x, conv.ins[1], dw.ins[1], pr.ins[1]], y,
                {"padded": ep}, {conv.ins[1]: [E, C], pr.ins[1]: [C, E]})


class Program:
    """The entry-point calls of a lowered function, run in order on torch
    tensors that live on the GPU."""

    def __init__(self, func: mlir.MFunc, calls: list):
        self.func = func
        self.calls = calls

    @property
    def entry_points(self):
        return [c.entry for c in self.calls]

    def run(self, inputs: dict, stream=None) -> dict:
        """inputs: argument name (with or without %) -> tensor.  Returns the
        function's results by SSA name."""
        import torch

        from . import groups

        vals = {}
        for a, _ in self.func.args:
            t = inputs.get(a, inputs.get(a.lstrip("%")))
            if t is None:
                raise KeyError(f"no tensor for argument {a}")
            vals[a] = t
        for c in self.calls:
            args = []
            for v in c.args:
                if v is None:
                    args.append(None)
                    continue
                t = vals[v]
                if v in c.views:
                    t = t.reshape(c.views[v])
                args.append(t)
            oty = self.func.types[c.out]
            dt = getattr(torch, _TORCH_DTYPE[oty.elem])
            out = torch.empty(oty.shape, dtype=dt, device=args[0].device)
            if c.entry == "fused_matmul_bias_act":
                groups.fused_matmul_bias_act(args[0], args[1], args[2], out, c.params["act"], stream)
            elif c.entry == "fused_conv2d_nhwc_bias_act":
                groups.fused_conv2d_nhwc_bias_act(args[0], args[1], args[2], out, c.params["pad"],
                                                  c.params["act"], stream)
            elif c.entry == "fused_irb_f32":
                groups.fused_irb_f32(args[0], args[1], args[2], args[3], out, stream)
            else:  # pragma: no cover - lower() emits only the entries above
                raise NotImplementedError(c.entry)
            vals[c.out] = out
        ret = [op for op in self.func.ops if op.name == "func.return"]
        names = ret[0].operands if ret else []
        return {n: vals[n] for n in names}


def lower_text(text: str, target=None) -> "Program":
    """`lower` on the first function of an MLIR text."""
    return lower(mlir.parse_functions(text)[0], target)
