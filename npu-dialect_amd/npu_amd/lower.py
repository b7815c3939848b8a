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
  bodies -> fused_matmul_bias_act (f32).  A group holding several matmul
  chains (test/mlp.mlir's matmul -> ReLU -> matmul -> ReLU) becomes one call
  per chain, in order;
* {fill, conv_2d_nhwc_fhwc, generic...}, its input optionally a tensor.pad of
  zeros symmetric in H and W -> fused_conv2d_nhwc_bias_act (f32 / bf16), the pad
  folded into the call; with a residual term in the generic (a ResNet block's
  add) -> fused_conv2d_nhwc_bias_res_act;
* {fill, conv_2d_nchw_fchw, generic...} -- the reference's own layout
  (test/conv2d_relu.mlir, test/resnet_block.mlir, test/resnet50_block.mlir,
  test/mobilenet_block.mlir), 1x1 or 3x3 -> fused_conv2d_nchw_bias_act (f32),
  the pad folded, or with the residual of an add generic (and a ReLU after it
  in a second generic) -> fused_conv2d_nchw_bias_res_act;
* the inverted residual chain: {fill, 1x1 conv, ReLU6 generic} -> tensor.pad ->
  depthwise 3x3 -> ReLU6 generic -> 1x1 conv -> generic adding the chain's
  input (one group after the pad, or two: the fusion decision depends on the
  shapes) -> one fused_irb_f32 call (f32), the expanded tensor never leaving
  the chip.

A generic is matched by what its region computes, not by the names of the ops
in it: the yielded value must be the chain's value plus, optionally, a bias
(indexing map: the last output dimension only) and a residual (identity map),
through `arith.addf`, then optionally `arith.maximumf(., 0.0)` (ReLU) and
`arith.minimumf(., 6.0)` on top of it (ReLU6); every `linalg.fill` and
`tensor.pad` must write 0.0.  Anything else -- an op no group covers, another
body, another dtype, a stride or dilation -- raises NotImplementedError naming
it: there is no fallback implementation.

f16 text is run the way the reference harness runs it: every `f16` of the text
becomes `f32` before anything else (tools/harness/e2e_verify.py:163-164), so
`lower_text` of test/matmul_relu.mlir executes the f32 function the
reference's CPU path executes.
"""
from __future__ import annotations

import re
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
    outs: list = None          # every result, when the entry point writes several


@dataclass
class Launch:
    """One npu_group_launch: the outlined group(s) by name, their external
    inputs in first-use order (SSA names), the result and the attributes."""
    name: str                  # outlined names joined by '+'
    ins: list                  # SSA names, the outlined function's argument order
    out: str
    acts: list                 # activation of each matmul/conv chain
    pad: int = 0               # > 0: the padded input `padded` is passed unpadded
    padded: str = None
    pad_source: str = None
    stores: list = field(default_factory=list)   # tensor.empty values holding intermediates
    widen: list = field(default_factory=list)    # bf16 biases passed widened to f32
    entry: str = "npu_group_launch"   # or a typed entry point taking `ins`, `outs`, `params`
    outs: list = None
    params: dict = field(default_factory=dict)
    res_arg: int = 0           # index of a conv group's residual in `ins` (0: none)
    stride: int = 1            # an NCHW conv group's stride


_TORCH_DTYPE = {"f32": "float32", "bf16": "bfloat16", "i8": "int8", "i32": "int32"}


def harness_f32(text: str) -> str:
    """The reference harness's element-type rule: the text's f16 becomes f32
    (tools/harness/e2e_verify.py:163-164, `original.replace('f16', 'f32')`).
    The reference's texts hold no bf16; here bf16 is left as it is."""
    return re.sub(r"(?<!b)f16", "f32", text)


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


def _float(literal):
    """The value of an arith.constant literal ("0.0", "6.000000e+00",
    "0xFF800000"), or None."""
    if literal is None:
        return None
    text = str(literal).split(":")[0].strip()
    if re.fullmatch(r"0x[0-9A-Fa-f]{8}", text):  # MLIR's f32 bit-pattern form (inf, nan)
        import struct

        return struct.unpack("<f", struct.pack("<I", int(text, 16)))[0]
    try:
        return float(text)
    except ValueError:
        return None


def _const(fn: _Fn, v):
    op = fn.op(v)
    if op is None or op.name != "arith.constant":
        return None
    return _float(op.attrs.get("value"))


def _body_value(g):
    """The yielded value of generic `g` as an expression: ("arg", k) for block
    argument k, ("const", x), or (op name, lhs, rhs) for a binary arith op."""
    args, body, yielded = g.attrs.get("block_args", []), g.attrs.get("body", []), \
        g.attrs.get("yield", [])
    env = {a: ("arg", k) for k, a in enumerate(args)}
    for b in body:
        if b.name == "arith.constant":
            env[b.result] = ("const", _float(b.value))
        elif b.name in ("arith.addf", "arith.maximumf", "arith.minimumf") and len(b.operands) == 2:
            if any(o not in env for o in b.operands):
                raise NotImplementedError(f"{g.results[0]}: generic body reads a value "
                                          f"defined outside it ({b.operands})")
            env[b.result] = (b.name, env[b.operands[0]], env[b.operands[1]])
        else:
            raise NotImplementedError(f"{g.results[0]}: {b.name} in a generic body "
                                      "(epilogues are addf / maximumf / minimumf)")
    if len(yielded) != 1 or yielded[0] not in env:
        raise NotImplementedError(f"{g.results[0]}: generic yields {yielded}")
    return env[yielded[0]]


def _tree(g):
    """The yielded value of generic `g` as a full expression tree: ("arg", k),
    ("const", literal, type) or (op name, type, operand trees...)."""
    args, body, yielded = g.attrs.get("block_args", []), g.attrs.get("body", []), \
        g.attrs.get("yield", [])
    env = {a: ("arg", k) for k, a in enumerate(args)}
    for b in body:
        if b.name == "arith.constant":
            env[b.result] = ("const", b.value, b.type)
        elif b.name == "linalg.index":
            env[b.result] = (b.name, b.type, ("dim", int(b.value)))
        elif b.name in ("arith.cmpi", "arith.cmpf"):
            if any(o not in env for o in b.operands):
                raise NotImplementedError(f"{g.results[0]}: generic body reads a value "
                                          f"defined outside it ({b.operands})")
            env[b.result] = (b.name, b.type, ("pred", b.value)) + tuple(env[o] for o in b.operands)
        else:
            if any(o not in env for o in b.operands):
                raise NotImplementedError(f"{g.results[0]}: generic body reads a value "
                                          f"defined outside it ({b.operands})")
            env[b.result] = (b.name, b.type) + tuple(env[o] for o in b.operands)
    if len(yielded) != 1 or yielded[0] not in env:
        raise NotImplementedError(f"{g.results[0]}: generic yields {yielded}")
    return env[yielded[0]]


_COMMUTATIVE = ("arith.addf", "arith.mulf", "arith.maximumf", "arith.minimumf",
                "arith.addi", "arith.muli")


def _matches(tree, tmpl, binds):
    """Structural match of an expression tree against a template whose leaves
    are ("$name",) placeholders (bound to one subtree each, consistently).
    The two operands of a commutative op (IEEE addition, multiplication,
    maximum and minimum give the same bits in either order) match in either
    order; nothing is reassociated."""
    if len(tmpl) == 1 and tmpl[0].startswith("$"):
        key = tmpl[0]
        if key in binds:
            return binds[key] == tree
        binds[key] = tree
        return True
    if tmpl[0] == "const":
        return tree[0] == "const" and _float(tree[1]) == _float(tmpl[1]) and tree[2] == tmpl[2]
    if len(tree) != len(tmpl) or tree[0] != tmpl[0] or tree[1] != tmpl[1]:
        return False
    orders = [tmpl[2:]]
    if tmpl[0] in _COMMUTATIVE and len(tmpl) == 4:
        orders.append((tmpl[3], tmpl[2]))
    for order in orders:
        trial = dict(binds)
        if all(_matches(a, b, trial) for a, b in zip(tree[2:], order)):
            binds.clear()
            binds.update(trial)
            return True
    return False


def _apply_scale_tmpl():
    """TOSA apply_scale_32, single rounding, in arith (i64), truncated to i32:
    trunci((extsi(acc) * extsi(m) + (1 << (extsi(s) - 1))) >> extsi(s))."""
    s64 = ("arith.extsi", "i32 to i64", ("$s",))
    one = ("const", "1", "i64")
    prod = ("arith.muli", "i64", ("arith.extsi", "i32 to i64", ("$acc",)),
            ("arith.extsi", "i32 to i64", ("$m",)))
    rnd = ("arith.shli", "i64", one, ("arith.subi", "i64", s64, one))
    return ("arith.trunci", "i64 to i32",
            ("arith.shrsi", "i64", ("arith.addi", "i64", prod, rnd), s64))


def _requant_of(fn: "_Fn", g, acc, shape):
    """(m, s, residual) when generic `g` computes the int8 requantization of
    accumulator `acc`: trunci(minsi(maxsi(apply_scale(acc) [+ extsi(x)], 0),
    127)) to i8, m and s per output channel (the last dimension), the
    residual x of the output's shape; else raises NotImplementedError."""
    rank = len(shape)
    ident = list(range(rank))
    name = g.results[0]
    maps = g.attrs.get("maps", [])
    if len(g.results) != 1 or g.iterators != ["parallel"] * rank or len(maps) != len(g.ins) + 1 \
            or maps[-1] != ident or not g.ins or g.ins[0] != acc or maps[0] != ident:
        raise NotImplementedError(f"{name}: not a requantization of {acc}")
    scale = _apply_scale_tmpl()
    for resid in (False, True):
        inner = ("arith.addi", "i32", scale, ("arith.extsi", "i8 to i32", ("$x",))) if resid else scale
        tmpl = ("arith.trunci", "i32 to i8",
                ("arith.minsi", "i32", ("arith.maxsi", "i32", inner, ("const", "0", "i32")),
                 ("const", "127", "i32")))
        b = {}
        if not _matches(_tree(g), tmpl, b):
            continue
        pos = {k: b[k][1] for k in b if b[k][0] == "arg"}
        if set(pos) != ({"$acc", "$m", "$s", "$x"} if resid else {"$acc", "$m", "$s"}) or \
                pos["$acc"] != 0:
            break
        m, sh = g.ins[pos["$m"]], g.ins[pos["$s"]]
        if maps[pos["$m"]] != [rank - 1] or maps[pos["$s"]] != [rank - 1]:
            break
        if fn.ty(m).shape != [shape[-1]] or fn.ty(sh).shape != [shape[-1]]:
            break
        x = None
        if resid:
            x = g.ins[pos["$x"]]
            if maps[pos["$x"]] != ident or fn.ty(x).shape != list(shape):
                break
        return m, sh, x
    raise NotImplementedError(f"{name}: generic body is not the int8 requantization "
                              "(apply_scale, optional residual, clamp to [0, 127])")


def _clamp(e, op, bound):
    """x when e is op(x, bound) or op(bound, x), else None."""
    if e[0] != op:
        return None
    a, b = e[1], e[2]
    if b == ("const", bound):
        return a
    if a == ("const", bound):
        return b
    return None


def _sum_leaves(e):
    if e[0] == "arith.addf":
        return _sum_leaves(e[1]) + _sum_leaves(e[2])
    return [e]


def _match_generic(fn: _Fn, g, v, shape, cdim=-1):
    """(bias, residual, act) of one epilogue generic applied to chain value v;
    a bias is indexed by the channel dimension `cdim` alone (the last for
    NHWC and matrices, 1 for NCHW)."""
    rank = len(shape)
    cdim = cdim % rank
    ident = list(range(rank))
    name = g.results[0]
    maps = g.attrs.get("maps", [])
    if len(g.results) != 1 or len(g.outs) != 1:
        raise NotImplementedError(f"{name}: generic with {len(g.results)} results")
    if g.iterators != ["parallel"] * rank:
        raise NotImplementedError(f"{name}: iterators {g.iterators} (epilogues are parallel)")
    if len(maps) != len(g.ins) + 1 or maps[-1] != ident:
        raise NotImplementedError(f"{name}: indexing maps {maps}")
    if v not in g.ins:
        raise NotImplementedError(f"{name}: epilogue not on the chain from {v}")
    e = _body_value(g)
    act = "none"
    inner = _clamp(e, "arith.minimumf", 6.0)
    if inner is not None:
        x = _clamp(inner, "arith.maximumf", 0.0)
        if x is None:
            raise NotImplementedError(f"{name}: minimumf(., 6.0) not over maximumf(., 0.0)")
        act, e = "relu6", x
    else:
        x = _clamp(e, "arith.maximumf", 0.0)
        if x is not None:
            act, e = "relu", x
    bias = residual = None
    seen_chain = False
    for leaf in _sum_leaves(e):
        if leaf[0] != "arg" or leaf[1] >= len(g.ins):
            raise NotImplementedError(f"{name}: generic body term {leaf} "
                                      "(a block argument of an input expected)")
        operand, m = g.ins[leaf[1]], maps[leaf[1]]
        t = fn.ty(operand)
        if operand == v and m == ident and not seen_chain:
            seen_chain = True
        elif m == [cdim] and t.shape == [shape[cdim]] and bias is None:
            bias = operand
        elif m == ident and t.shape == list(shape) and residual is None:
            residual = operand
        else:
            raise NotImplementedError(f"{name}: operand {operand} {t} with map {m} "
                                      "in the epilogue")
    if not seen_chain:
        raise NotImplementedError(f"{name}: the chain value {v} is not a term of the result")
    return bias, residual, act


def _epilogue(fn: _Fn, generics, src, shape, cdim=-1):
    """Bias, residual and activation of the generics that follow `src` in a
    group, applied in order; returns (bias, residual, act, last value)."""
    bias = residual = None
    act = "none"
    v = src
    for g in generics:
        b, r, a = _match_generic(fn, g, v, shape, cdim)
        if act != "none" and (b or r or a != "none"):
            raise NotImplementedError(f"{g.results[0]}: epilogue after the activation")
        if b is not None:
            if bias is not None or residual is not None:
                raise NotImplementedError(f"{g.results[0]}: a second bias / bias after a residual")
            bias = b
        if r is not None:
            if residual is not None:
                raise NotImplementedError(f"{g.results[0]}: a second residual")
            residual = r
        act = a if a != "none" else act
        v = g.results[0]
    return bias, residual, act, v


def _check_fill(fn: _Fn, fill):
    if fill.ins and fill.ins[0] in {a for a, _ in fn.f.args}:
        return  # an outlined kernel's argument: npu_group_launch checks its value
    c = _const(fn, fill.ins[0]) if fill.ins else None
    if c != 0.0:
        raise NotImplementedError(f"{fill.results[0]}: linalg.fill with {fill.ins} "
                                  "(accumulators start at 0.0)")


def _pad_of(fn: _Fn, v, nchw=False):
    """(source, pad) when v is a tensor.pad of zeros by p in H and W only
    (dimensions 1 and 2 of NHWC, 2 and 3 of NCHW)."""
    op = fn.op(v)
    if op is None or op.name != "tensor.pad":
        return v, 0
    lo, hi = op.attrs.get("low", []), op.attrs.get("high", [])
    h, w_ = (2, 3) if nchw else (1, 2)
    if (len(lo) != 4 or lo != hi or lo[h] != lo[w_]
            or any(lo[d] for d in range(4) if d not in (h, w_))):
        raise NotImplementedError(f"{v}: pad low {lo} high {hi} (entry points pad H and W equally)")
    if _const(fn, op.attrs.get("yield")) != 0.0:
        raise NotImplementedError(f"{v}: tensor.pad yields {op.attrs.get('yield')} (zero padding)")
    return op.operands[0], lo[h]


def _check_conv(op, strided=False):
    """The conv's stride (refused unless `strided`: the NCHW entry points
    take one stride for both spatial dimensions); dilations must be 1."""
    st = op.attrs.get("strides", [1, 1])
    if any(s != 1 for s in st) and (not strided or len(set(st)) != 1):
        raise NotImplementedError(f"{op.results[0]}: strided convolution {st}")
    if "dilations" in op.text and "dilations = dense<1>" not in op.text.replace("  ", " "):
        raise NotImplementedError(f"{op.results[0]}: dilated convolution")
    return st[0] if st else 1


def _check_matmul(op):
    if "indexing_maps" in op.text:
        raise NotImplementedError(f"{op.results[0]}: linalg.matmul with indexing maps")


def _elem(fn, v, allowed, what):
    e = fn.ty(v).elem
    if e not in allowed:
        raise NotImplementedError(f"{what}: element type {e} (entry point takes {'/'.join(allowed)})")
    return e


ANCHORS = ("linalg.matmul", "linalg.conv_2d_nhwc_fhwc", "linalg.conv_2d_nchw_fchw")


def _segments(name, ops):
    """Splits a group's ops into chains [fills..., anchor, generics...]: each
    fill goes with the anchor whose accumulator it initialises, each generic
    with the chain whose value it reads."""
    anchors = [o for o in ops if o.name in ANCHORS]
    if not anchors:
        raise NotImplementedError(f"{name}: no MI355X entry point runs ops "
                                  f"{[o.name for o in ops if o.name != 'linalg.fill']}")
    segs = [{"anchor": a, "fills": [], "generics": [], "value": a.results[0]} for a in anchors]
    for o in ops:
        if o.name in ANCHORS:
            continue
        if o.name == "linalg.fill":
            owner = [s for s in segs if o.results[0] in s["anchor"].outs]
            if len(owner) != 1:
                raise NotImplementedError(f"{name}: {o.results[0]} fills no accumulator")
            owner[0]["fills"].append(o)
        elif o.name == "linalg.generic":
            owner = [s for s in segs if s["value"] in o.ins]
            if not owner:
                raise NotImplementedError(f"{name}: {o.results[0]} is on no matmul/conv chain")
            # a generic joining two chains of the group (a ResNet block's add of
            # its shortcut conv) continues the later one; the earlier chain's
            # value is then its residual operand
            owner = max(owner, key=lambda s: ops.index(s["anchor"]))
            owner["generics"].append(o)
            owner["value"] = o.results[0]
        else:
            raise NotImplementedError(f"{name}: no MI355X entry point runs {o.name} in a group")
    for s in segs:
        if len(s["fills"]) != 1:
            raise NotImplementedError(f"{name}: {s['anchor'].results[0]} accumulates into a "
                                      "value that is not a fill of 0.0")
    return segs


def lower(func: mlir.MFunc, target=None, groups=None) -> "Program":
    """Matches func's outlined groups to entry points; see the module docstring.
    `groups` ([{name, ops, inputs, outputs}], ops as indices into func.ops)
    gives the groups instead of the restated pipeline's decisions: the
    outlined kernels of a module npu-opt has already run (npu_amd.reader)."""
    from . import lower_llama

    fn = _Fn(func)
    if groups is None:
        rep = pipeline.run(func, target)
    else:
        inside = {i for g in groups for i in g["ops"]}
        rest = [i for i, o in enumerate(func.ops) if o.name.startswith("linalg.")
                and i not in inside]
        rep = {"functions": [dict(g) for g in groups] +
               ([{"name": func.name, "ops": rest, "inputs": [], "outputs": []}] if rest else [])}
    groups = {g["name"]: [func.ops[i] for i in g["ops"]] for g in rep["functions"]}
    calls, covered, consumed, dests = [], set(), set(), {}
    # a Llama layer: its calls span the pipeline's groups, which hold only its ops
    llama = lower_llama.llama_calls(fn)
    in_llama = {r for c in llama for o in c["ops"] for r in o.results}
    for c in llama:
        names = [n for n, ops in groups.items() if n != func.name
                 and any(r in in_llama and any(r in o.results for o in c["ops"])
                        for op in ops for r in op.results)]
        calls.append(Call(c["entry"], names, c["args"], c["outs"][-1], c["params"],
                          outs=c["outs"]))
    covered |= in_llama
    for name, ops in groups.items():
        if name in consumed:
            continue
        inside = [r for o in ops if o.name != "linalg.fill" for r in o.results]
        if inside and all(r in in_llama for r in inside):
            continue
        if any(r in in_llama for r in inside):
            raise NotImplementedError(f"{name}: group mixes the Llama layer's ops with others")
        segs = _segments(name, ops)
        for s in segs:
            _check_fill(fn, s["fills"][0])
            a = s["anchor"]
            shape = fn.ty(a.results[0]).shape
            if a.name != "linalg.matmul" and fn.ty(a.ins[0]).elem == "i8":
                _check_conv(a)
                chain = _qbottleneck_chain(fn, groups, name, segs)
                calls.append(chain)
                consumed.update(chain.functions)
                covered.update(r for f2 in chain.functions for o in groups[f2] for r in o.results)
                covered.update(fn.op(chain.params["padded"]).results)
                break
            nchw = a.name == "linalg.conv_2d_nchw_fchw"
            bias, res, act, out = _epilogue(fn, s["generics"], a.results[0], shape,
                                            1 if nchw else -1)
            if nchw:
                stride = _check_conv(a, strided=True)
                x, pad = _pad_of(fn, a.ins[0], nchw=True)
                _elem(fn, x, ("f32",), name)
                for v in (bias, res):
                    if v is not None and fn.ty(v).elem != "f32":
                        raise NotImplementedError(f"{name}: {v} of type {fn.ty(v).elem}")
                params = {"pad": pad, "act": act, "stride": stride}
                if res is not None:
                    calls.append(Call("fused_conv2d_nchw_bias_res_act", [name],
                                      [x, a.ins[1], bias, res], out, params))
                else:
                    calls.append(Call("fused_conv2d_nchw_bias_act", [name], [x, a.ins[1], bias],
                                      out, params))
                if pad:
                    covered.add(a.ins[0])
                covered.update(r for o in ops for r in o.results)
                continue
            if a.name == "linalg.matmul":
                _check_matmul(a)
                if res is not None:
                    raise NotImplementedError(f"{name}: residual add after a matmul")
                _elem(fn, a.ins[0], ("f32",), name)
                calls.append(Call("fused_matmul_bias_act", [name], [a.ins[0], a.ins[1], bias], out,
                                  {"act": act}))
                dests[id(calls[-1])] = (s["generics"][-1].outs[0] if s["generics"]
                                        else s["fills"][0].outs[0])
                continue
            _check_conv(a)
            x, pad = _pad_of(fn, a.ins[0])
            # the expand group of an inverted residual chain: fold the chain
            chain = _irb_chain(fn, groups, name, a, out, x, act, bias, res) if len(segs) == 1 \
                else None
            if chain is not None:
                calls.append(chain)
                consumed.update(chain.functions)
                covered.update(r for f2 in chain.functions for o in groups[f2] for r in o.results)
                covered.update(fn.op(chain.params["padded"]).results)
                continue
            e = _elem(fn, x, ("f32", "bf16"), name)
            params = {"pad": pad, "act": act}
            if bias is not None and fn.ty(bias).elem != "f32":
                if fn.ty(bias).elem != e:
                    raise NotImplementedError(f"{name}: bias type {fn.ty(bias).elem}")
                params["bias_to_f32"] = True  # exact widening; the group adds in f32
            if res is not None:
                if fn.ty(res).elem != e:
                    raise NotImplementedError(f"{name}: residual type {fn.ty(res).elem}")
                calls.append(Call("fused_conv2d_nhwc_bias_res_act", [name],
                                  [x, a.ins[1], bias, res], out, params))
            else:
                calls.append(Call("fused_conv2d_nhwc_bias_act", [name], [x, a.ins[1], bias], out,
                                  params))
            if pad:
                covered.add(a.ins[0])
        covered.update(r for o in ops for r in o.results)
    # every computing op must be part of a call
    for op in func.ops:
        if op.name.startswith("linalg.") or op.name in ("tensor.pad", "tensor.expand_shape",
                                                          "tensor.collapse_shape"):
            if not op.results or op.results[0] not in covered:
                raise NotImplementedError(f"{op.results[0] if op.results else op.name}: "
                                          f"{op.name} is in no group an entry point runs")
    # dataflow order: a call runs after the calls whose results it reads
    pos = {r: i for i, op in enumerate(func.ops) for r in op.results}
    calls.sort(key=lambda c: max(pos[v] for v in (c.outs or [c.out])))
    return Program(func, calls, _launches(fn, rep, calls, dests))


def _launches(fn: _Fn, rep, calls, dests):
    """Groups the calls into npu_group_launch calls: consecutive calls of the
    same outlined functions are one launch (a group of several matmul chains);
    a call spanning several groups (the inverted residual chain) is one
    launch of their '+'-joined names."""
    by_name = {f["name"]: f for f in rep["functions"]}
    per_group = {}
    for c in calls:
        per_group[tuple(c.functions)] = per_group.get(tuple(c.functions), 0) + 1
    out, i = [], 0
    while i < len(calls):
        c = calls[i]
        if c.outs is not None:  # a typed Llama entry point
            out.append(Launch("+".join(c.functions), list(c.args), c.out, [], entry=c.entry,
                              outs=list(c.outs), params=dict(c.params)))
            i += 1
            continue
        if c.entry.startswith("fused_conv2d_nchw") and per_group[tuple(c.functions)] > 1:
            # an NCHW group of several conv chains (a ResNet downsampling
            # block's shortcut and second conv): each chain through its typed
            # entry point, in dataflow order
            out.append(Launch("+".join(c.functions), list(c.args), c.out, [], entry=c.entry,
                              outs=[c.out], params=dict(c.params)))
            i += 1
            continue
        j = i + 1
        while j < len(calls) and calls[j].functions == calls[i].functions:
            j += 1
        cs = calls[i:j]
        names = cs[0].functions
        inside = set()
        for n in names:
            for k in by_name[n]["ops"]:
                inside.update(fn.f.ops[k].results)
        padded = cs[0].params.get("padded")
        if padded:
            inside.add(padded)
        ins = []
        for n in names:
            for v in by_name[n]["inputs"]:
                if v not in inside and v not in ins:
                    ins.append(v)
        L = Launch("+".join(names), ins, cs[-1].out,
                   [c.params.get("act", "none") for c in cs])
        L.stride = cs[0].params.get("stride", 1)
        c0 = cs[0]
        if c0.entry.startswith("fused_conv2d_n") and c0.params.get("pad"):
            conv_in = [v for v in ins if fn.op(v) is not None and fn.op(v).name == "tensor.pad"]
            L.pad, L.padded, L.pad_source = c0.params["pad"], conv_in[0], c0.args[0]
        if c0.params.get("bias_to_f32"):
            L.widen.append(c0.args[2])
        L.stores = [dests[id(c)] for c in cs[:-1]]
        if c0.entry.endswith("_res_act"):  # the residual operand, by its argument index
            L.res_arg = ins.index(c0.args[3])
        out.append(L)
        i = j
    return out


def _qbottleneck_chain(fn, groups, name, segs):
    """The call running an int8 bottleneck chain whose first group is `name`:
    1x1 conv -> requant -> tensor.pad (zeros, 1 in H and W) -> 3x3 conv ->
    requant -> 1x1 conv -> requant + the chain's input -> fused_qbottleneck_i8,
    the intermediates never leaving the chip.  Raises NotImplementedError for
    any other int8 group."""
    if len(segs) != 1 or len(segs[0]["generics"]) != 1:
        raise NotImplementedError(f"{name}: int8 group other than conv -> requant")
    c1, g1 = segs[0]["anchor"], segs[0]["generics"][0]
    _check_fill(fn, segs[0]["fills"][0])
    x, w1 = c1.ins
    xs = fn.ty(x).shape
    if fn.ty(w1).shape[1:3] != [1, 1] or fn.ty(x).elem != "i8" or fn.ty(w1).elem != "i8":
        raise NotImplementedError(f"{name}: int8 chain must start with a 1x1 conv of int8 values")
    m1, s1, r1 = _requant_of(fn, g1, c1.results[0], fn.ty(c1.results[0]).shape)
    y1 = g1.results[0]

    def user(v, kind):
        us = [o for o in fn.f.ops if o.name == kind and (v in o.ins or v in o.operands)]
        if len(us) != 1:
            raise NotImplementedError(f"{v}: expected one {kind} user")
        return us[0]

    pad = user(y1, "tensor.pad")
    src, p = _pad_of(fn, pad.results[0])
    if p != 1 or src != y1:
        raise NotImplementedError(f"{pad.results[0]}: the 3x3 conv's pad must be 1 in H and W")
    c2 = user(pad.results[0], "linalg.conv_2d_nhwc_fhwc")
    _check_conv(c2)
    g2 = user(c2.results[0], "linalg.generic")
    m2, s2, r2 = _requant_of(fn, g2, c2.results[0], fn.ty(c2.results[0]).shape)
    c3 = user(g2.results[0], "linalg.conv_2d_nhwc_fhwc")
    _check_conv(c3)
    g3 = user(c3.results[0], "linalg.generic")
    m3, s3, r3 = _requant_of(fn, g3, c3.results[0], fn.ty(c3.results[0]).shape)
    if r1 is not None or r2 is not None or r3 != x:
        raise NotImplementedError(f"{g3.results[0]}: the residual must be the chain's input only")
    w2, w3 = c2.ins[1], c3.ins[1]
    M1 = fn.ty(w1).shape[0]
    if fn.ty(w2).shape != [M1, 3, 3, M1] or fn.ty(w3).shape != [xs[3], 1, 1, M1]:
        raise NotImplementedError(f"{name}: filter shapes {fn.ty(w2).shape} {fn.ty(w3).shape}")
    group_of = {o.results[0]: n for n, ops in groups.items() for o in ops if o.results}
    names = []
    for o in (c1, g1, c2, g2, c3, g3):
        n = group_of.get(o.results[0])
        if n is None:
            raise NotImplementedError(f"{o.results[0]} is in no outlined group")
        if n not in names:
            names.append(n)
    chain_ops = {id(o) for o in (c1, g1, c2, g2, c3, g3)}
    for n in names:
        for o in groups[n]:
            if o.name == "linalg.fill":
                _check_fill(fn, o)
            elif id(o) not in chain_ops:
                raise NotImplementedError(f"{n}: {o.name} in the int8 chain")
    C = xs[3]
    return Call("fused_qbottleneck_i8", names, [x, w1, w2, w3, m1, s1, m2, s2, m3, s3],
                g3.results[0], {"padded": pad.results[0]}, {w1: [M1, C], w3: [C, M1]})


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
    if g2 is None or (b1, r1, a1) != (None, None, "relu6"):
        return None
    _check_conv(dw)
    _check_conv(pr)
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
    # the chain's groups hold only these ops (and fills of 0.0)
    chain_ops = {id(o) for o in (dw, g1, pr, g2)}
    for n in names[1:]:
        for o in groups[n]:
            if o.name == "linalg.fill":
                _check_fill(fn, o)
            elif id(o) not in chain_ops:
                return None
    _elem(fn, x, ("f32",), names[-1])
    E, C = wshape[0], wshape[3]
    return Call("fused_irb_f32", names, [x, conv.ins[1], dw.ins[1], pr.ins[1]], y,
                {"padded": ep}, {conv.ins[1]: [E, C], pr.ins[1]: [C, E]})


class Program:
    """The entry-point calls of a lowered function, run in order on torch
    tensors that live on the GPU."""

    def __init__(self, func: mlir.MFunc, calls: list, launches: list = ()):
        self.func = func
        self.calls = calls
        self.launches = list(launches)

    @property
    def entry_points(self):
        return [c.entry for c in self.calls]

    def check_inputs(self, inputs: dict) -> dict:
        """Binds every argument to its tensor and checks the tensor's dtype and
        shape against the function's signature."""
        import torch

        vals = {}
        for a, t in self.func.args:
            x = inputs.get(a, inputs.get(a.lstrip("%")))
            if x is None:
                raise KeyError(f"no tensor for argument {a}")
            want = getattr(torch, _TORCH_DTYPE.get(t.elem, "void"), None)
            if x.dtype != want:
                raise TypeError(f"argument {a}: tensor of {x.dtype}, the function takes {t}")
            if list(x.shape) != list(t.shape):
                raise ValueError(f"argument {a}: tensor of shape {list(x.shape)}, "
                                 f"the function takes {t}")
            vals[a] = x
        return vals

    def run_launch(self, index: int, vals: dict, stream=None):
        """Runs launch `index` on the values bound so far (function arguments
        and earlier launches' results, by SSA name) and binds its result."""
        import torch

        from . import groups

        L = self.launches[index]
        types = self.func.types
        tdt = lambda e: getattr(torch, _TORCH_DTYPE[e])
        dev = next(iter(vals.values())).device
        if L.entry != "npu_group_launch":
            for v in L.outs:
                if v not in vals:
                    vals[v] = torch.empty(types[v].shape, dtype=tdt(types[v].elem), device=dev)
            ins = [None if v is None else vals[v] for v in L.ins]
            outs = [vals[v] for v in L.outs]
            getattr(groups, L.entry)(*ins, *outs, **L.params, stream=stream)
            return
        prod = {r: op for op in self.func.ops for r in op.results}
        ins = []
        for v in L.ins:
            op = prod.get(v)
            if v == L.padded:
                ins.append(vals[L.pad_source])
            elif v in vals:
                t = vals[v]
                ins.append(t.float() if v in L.widen else t)
            elif op is not None and op.name == "arith.constant":
                ins.append(_float(op.attrs.get("value")))
            elif op is not None and op.name == "tensor.empty":
                t = types[v]
                keep = torch.empty(t.shape, dtype=tdt(t.elem), device=dev) \
                    if v in L.stores else None
                ins.append(groups.Empty(t.shape, t.elem, keep))
            else:  # pragma: no cover - lower() binds every input
                raise KeyError(f"{L.name}: no value for {v}")
        oty = types[L.out]
        if L.out not in vals:
            vals[L.out] = torch.empty(oty.shape, dtype=tdt(oty.elem), device=dev)
        groups.group_launch(L.name, ins, [vals[L.out]], act=L.acts, pad=L.pad, stream=stream,
                            res_arg=L.res_arg, stride=L.stride)

    def run(self, inputs: dict, stream=None) -> dict:
        """inputs: argument name (with or without %) -> tensor.  Runs every
        launch through npu_group_launch and returns the function's results by
        SSA name."""
        vals = self.check_inputs(inputs)
        for i in range(len(self.launches)):
            self.run_launch(i, vals, stream)
        ret = [op for op in self.func.ops if op.name == "func.return"]
        names = ret[0].operands if ret else []
        return {n: vals[n] for n in names}


def cost_report(program: "Program", inputs: dict, reps: int = 20, stream=None) -> list:
    """The pipeline's COST_JSON records of the program's outlined functions
    (CostEvaluatePass.cpp:135-158, the reference's keys in its order) with
    what the MI355X adds after them: the entry point that runs the function,
    the launch model's prediction for that launch (``mi355x_predicted_us``,
    from the launch plans the entry point records) and the launch's measured
    device time (``measured_us``: `reps` launches back to back between HIP
    events, queued behind a stream hold so that only device work is timed).
    A launch that runs several outlined functions (a chain fused across a
    tensor.pad) reports its figures on each of them, with its name."""
    import json

    import torch

    from . import groups, host

    rep = pipeline.run(program.func)
    records = {f["name"]: json.loads(line[len("COST_JSON: "):])
               for f, line in zip(rep["functions"], rep["cost_json"])}
    out = []
    vals = program.check_inputs(inputs)
    for li, L in enumerate(program.launches):
        def one():
            program.run_launch(li, vals, stream)
        with groups.collect_plans() as cp:
            one()
        torch.cuda.synchronize()
        pred, _ = host.predict_block(cp.plans)
        st = torch.cuda.current_stream() if stream is None else stream
        torch.cuda._sleep(2_000_000)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        for _ in range(reps):
            one()
        b.record(st)
        torch.cuda.synchronize()
        meas = a.elapsed_time(b) * 1e3 / reps
        for name in L.name.split("+"):
            r = dict(records[name])
            r.update({"entry_point": L.entry if L.entry != "npu_group_launch"
                      else (L.name if "+" in L.name else name),
                      "mi355x_predicted_us": round(pred, 3), "measured_us": round(meas, 3)})
            out.append("COST_JSON: " + json.dumps(r))
    return out


def lower_text(text: str, target=None) -> "Program":
    """`lower` on the first function of an MLIR text, after the harness's
    f16 -> f32 rule."""
    return lower(mlir.parse_functions(harness_f32(text))[0], target)
