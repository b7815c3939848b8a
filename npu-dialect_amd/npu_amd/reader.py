"""Reads what npu-opt emits and runs it on the MI355X.

After the reference's pipeline (lib/Transforms/Pipeline.cpp:11-38) a module is
outlined kernels ``func.func private @fused_<ops>_<idx>(...) attributes
{npu.fused_kernel}`` (OutlineFusedGroupsPass.cpp:259-303) called from the
parent function -- inside a tile-and-fuse loop when fusion tiled the group
(FusionPass.cpp:306-359) -- and every function's linalg ops are spatially and
temporally tiled (`scf.for` nests over `tensor.extract_slice` /
`tensor.insert_slice`, peeled remainders; SpatialTilingPass.cpp:138-166,
TemporalTilingPass.cpp:308-333).  After npu-bufferize the same nests work on
memrefs: slices are `memref.subview`s, and every buffer a loop reads from
outside is staged through `npu.alloc_sram` + `npu.dma_copy` (written back by
a second dma_copy when the loop writes it; BufferizePass.cpp:97-222).

On the MI355X the whole nest of a group is one launch.  ``flatten`` reads a
module in either form and undoes the tiling: every tile of an op writes a
slice of one full destination, so each op of the untiled function is the op
applied to the full tensors its slices come from; the tiles of one op --
the loop body and its peeled remainders, the K steps that accumulate into
the same destination -- are recognised as one op (same op, same full inputs,
writing the result of that same op).  A DMA copy into SRAM makes the SRAM
buffer stand for the DRAM buffer it copies (the kernel reads LDS, the values
are the DRAM tensor's), and a copy back is the write of that tensor.
``func.call`` of an outlined kernel is inlined at full size, and the ops that
came from each kernel are kept as that kernel's group.

``lower_module`` then hands the untiled function to the host lowering with the
module's own groups (``lower.lower``), so each outlined kernel's loop nest
becomes one npu_group_launch (or a typed entry point) named by the kernel.
"""
from __future__ import annotations

import copy
import re
from dataclasses import dataclass, field

from . import mlir

INDEX_OPS = ("arith.subi", "arith.addi", "arith.muli", "arith.divui", "arith.divsi",
             "arith.remui", "arith.index_cast", "affine.apply", "affine.min", "affine.max",
             "npu.sync", "npu.barrier", "npu.dealloc_sram", "memref.dealloc", "arith.cmpi",
             "npu.core_yield")


@dataclass
class Node:
    name: str
    results: list
    text: str
    body: list = None          # scf.for / npu.core_execute region
    header: str = ""
    rest: str = ""             # the statement after its results


def _split_results(s):
    m = re.match(r"^\s*((?:%[\w]+(?::\d+)?\s*,\s*)*%[\w]+(?::\d+)?)\s*=\s*", s)
    if not m:
        return [], s.strip()
    res = []
    for r in m.group(1).split(","):
        r = r.strip()
        if ":" in r:
            base, n = r.split(":")
            res += [f"{base}#{k}" for k in range(int(n))]
        else:
            res.append(r)
    return res, s[m.end():].strip()


def parse_block(body: str) -> list:
    """The statements of a block, scf.for / npu.core_execute regions parsed
    recursively."""
    out = []
    for st in mlir._statements(body):
        res, rest = _split_results(st)
        name = re.match(r"[\w\.]+", rest).group(0)
        if name in ("scf.for", "npu.core_execute"):
            k = rest.index("{")
            e = rest.rindex("}")
            out.append(Node(name, res, st, parse_block(rest[k + 1:e]), rest[:k], rest))
        else:
            out.append(Node(name, res, st, rest=rest))
    return out


@dataclass
class Flat:
    """The untiled function: ops (mlir.MOp), types, and for each op index the
    outlined kernel it came from (None for the parent's own ops)."""
    func: mlir.MFunc
    group_of: list = field(default_factory=list)
    calls: list = field(default_factory=list)       # kernel names in call order


class _Flattener:
    def __init__(self, funcs):
        self.funcs = {f["name"]: f for f in funcs}
        self.ops, self.types, self.group_of = [], {}, []
        self.sig = {}             # flat value -> signature of the op that wrote it
        self.n = 0
        self.calls = []
        self.cur_group = None

    def fresh(self):
        self.n += 1
        return f"%v{self.n}"

    def add(self, op, group=None):
        self.ops.append(op)
        self.group_of.append(group if group is not None else self.cur_group)
        for r, t in zip(op.results, op.result_types):
            self.types[r] = t

    # ---------------------------------------------------------------- environment
    # env maps a local SSA name to ("t", flat tensor name) or ("b", root id);
    # roots map to their current flat tensor version.
    def tensor_of(self, env, v):
        k = env.get(v)
        if k is None:
            raise NotImplementedError(f"reader: {v} is not defined")
        if k[0] == "t":
            return k[1]
        return self.version(k[1])

    def version(self, root):
        cur = self.roots[root]["version"]
        if cur is None:
            t = self.roots[root]["type"]
            r = self.fresh()
            self.add(mlir.MOp("tensor.empty", [r], [t], text=f"{r} = tensor.empty() : {t}"))
            self.roots[root]["version"] = r
            cur = r
        return cur

    def new_root(self, t, version=None):
        rid = len(self.roots)
        self.roots.append({"type": mlir.TType(t.shape, t.elem), "version": version})
        return rid

    # ---------------------------------------------------------------- walking
    def run_function(self, fname, env):
        f = self.funcs[fname]
        self.roots = getattr(self, "roots", [])
        return self.block(parse_block(f["body"]), env)

    def block(self, nodes, env):
        """Processes nodes; returns the values of a terminator (scf.yield /
        return) as env entries."""
        for nd in nodes:
            r = self.node(nd, env)
            if r is not None:
                return r
        return None

    def node(self, nd, env):
        n = nd.name
        text = nd.rest.strip()
        if n in ("func.return", "return", "scf.yield"):
            vals = re.findall(r"%[\w#]+", text.split(":")[0])
            return [env[v] for v in vals]
        if n == "scf.for":
            m = re.search(r"iter_args\((.*?)\)\s*->", nd.header, re.S)
            inner = dict(env)
            if m:
                for pair in mlir._split_top(m.group(1)):
                    a, b = (x.strip() for x in pair.split("="))
                    inner[a] = env[b]
            ys = self.block(nd.body, inner) or []
            for r, y in zip(nd.results, ys):
                env[r] = y
            return None
        if n == "npu.core_execute":
            self.block(nd.body, env)
            return None
        if n == "arith.constant":
            ty = text.rsplit(":", 1)[1].strip()
            if ty == "index" or ty.startswith("i64") and "npu.core_id" in text:
                return None
            op = mlir.parse_op(text)
            r = self.fresh()
            op.results = [r]
            op.text = _rename_result(text, r)
            self.add(op, group=None)
            env[nd.results[0]] = ("t", r)
            return None
        if n in INDEX_OPS or n.startswith("npu.core"):
            return None
        if n == "tensor.empty":
            op = mlir.parse_op(text)
            r = self.fresh()
            op.results = [r]
            op.text = _rename_result(text, r)
            self.add(op, group=None)
            env[nd.results[0]] = ("t", r)
            return None
        if n in ("tensor.extract_slice", "memref.subview", "memref.cast",
                 "memref.reinterpret_cast", "tensor.cast"):
            src = re.match(r"[\w\.]+\s+(%[\w#]+)", text).group(1)
            env[nd.results[0]] = env[src]
            return None
        if n == "tensor.insert_slice":
            src = re.match(r"tensor\.insert_slice\s+(%[\w#]+)", text).group(1)
            env[nd.results[0]] = env[src]
            return None
        if n in ("memref.alloc", "memref.alloca"):
            t = mlir.parse_type(text.rsplit(":", 1)[1])
            env[nd.results[0]] = ("b", self.new_root(t))
            return None
        if n == "npu.alloc_sram":
            t = mlir.parse_type(text.rsplit(":", 1)[1])
            env[nd.results[0]] = ("b", self.new_root(t))
            return None
        if n == "npu.dma_copy":
            m = re.match(r"npu\.dma_copy\s+(%[\w#]+)\s+to\s+(%[\w#]+)\s+dir\s+(\w+)", text)
            a, b, d = m.groups()
            ka, kb = env[a], env[b]
            if d == "dram_to_sram":
                env[b] = ka if ka[0] == "b" else ("b", self.new_root(self.types[ka[1]], ka[1]))
            elif kb[0] == "b" and (ka[0] != "b" or ka[1] != kb[1]):
                self.roots[kb[1]]["version"] = self.tensor_of(env, a)
            return None
        if n == "memref.copy":
            a, b = re.findall(r"%[\w#]+", text.split(":")[0])[:2]
            kb = env[b]
            self.roots[kb[1]]["version"] = self.tensor_of(env, a)
            return None
        if n in ("bufferization.to_tensor",):
            src = re.match(r"[\w\.]+\s+(%[\w#]+)", text).group(1)
            env[nd.results[0]] = ("t", self.tensor_of(env, src))
            return None
        if n in ("bufferization.to_buffer", "bufferization.to_memref"):
            src = re.match(r"[\w\.]+\s+(%[\w#]+)", text).group(1)
            t = self.types[self.tensor_of(env, src)]
            env[nd.results[0]] = ("b", self.new_root(t, self.tensor_of(env, src)))
            return None
        if n == "func.call":
            return self.call(nd, env)
        if n.startswith("linalg."):
            return self.linalg(nd, env)
        if n in ("tensor.pad", "tensor.collapse_shape", "tensor.expand_shape"):
            op = mlir.parse_op(text)
            names = list(op.all_operands)
            if n == "tensor.pad" and op.attrs.get("yield"):
                names.append(op.attrs["yield"])  # the padding value, defined outside
            t2 = text
            for v in sorted(set(names), key=len, reverse=True):
                if v in env:
                    t2 = re.sub(re.escape(v) + r"(?![\w])", self.tensor_of(env, v), t2)
            r = self.fresh()
            op = mlir.parse_op(_rename_result(t2, r))
            op.text = _rename_result(t2, r)
            self.add(op)
            env[nd.results[0]] = ("t", r)
            return None
        if nd.results:
            raise NotImplementedError(f"reader: no rule for {n}")
        return None

    def call(self, nd, env):
        m = re.match(r"func\.call\s+@([\w]+)\(([^)]*)\)", nd.rest.strip())
        callee, args = m.group(1), [a.strip() for a in m.group(2).split(",") if a.strip()]
        if callee not in self.funcs:
            # a function this text does not hold: its results are opaque values
            rt = nd.rest.rsplit("->", 1)[1]
            rt = rt.strip()
            if rt.startswith("("):
                rt = rt[1:-1]
            for r, t in zip(nd.results, mlir._split_top(rt)):
                tt = mlir.parse_type(t)
                env[r] = ("t", self._opaque(tt))
            return None
        f = self.funcs[callee]
        inner = {}
        for (a, _), v in zip(f["args"], args):
            inner[a] = env[v]
        prev = self.cur_group
        if "npu.fused_kernel" in f["header"]:
            self.cur_group = callee
            if callee not in self.calls:
                self.calls.append(callee)
        ys = self.block(parse_block(f["body"]), inner) or []
        self.cur_group = prev
        for r, y in zip(nd.results, ys):
            env[r] = y
        return None

    def _opaque(self, tt):
        r = self.fresh()
        self.add(mlir.MOp("tensor.empty", [r], [tt], text=f"{r} = tensor.empty() : {tt}"))
        return r

    def linalg(self, nd, env):
        text = nd.text.strip()
        op = mlir.parse_op(text)
        memref = bool(re.search(r"outs\([^)]*:\s*memref<", text))
        ins = []
        for v in op.ins:
            k = env.get(v)
            ins.append(self.tensor_of(env, v) if k is not None else v)
        ov = op.outs[0]
        cur = self.tensor_of(env, ov)
        region = text[text.find("^bb"):text.rfind("}") + 1] if "^bb" in text else ""
        attrs = re.sub(r"\{?\s*barrier_gen = \d+ : i64, barrier_group = \d+ : i64\s*,?\s*\}?", "",
                       text.split("ins(")[0])
        sig = (op.name, region, re.sub(r"%[\w#]+|\s", "", attrs), tuple(ins))
        if self.sig.get(cur) == sig:
            r = cur  # another tile of the op that wrote `cur`
        else:
            r = self.fresh()
            full = copy.copy(op)
            full.ins = ins
            full.outs = [cur]
            full.results = [r]
            full.result_types = [self.types[cur]]
            full.attrs = dict(op.attrs)
            full.attrs["in_types"] = [self.types.get(v, mlir.TType([], "f32", False)) for v in ins]
            full.attrs["out_types"] = [self.types[cur]]
            full.text = _clean_attrs(text)
            self.add(full)
            self.sig[r] = sig
        if memref:
            k = env[ov]
            self.roots[k[1]]["version"] = r
        else:
            env[nd.results[0]] = ("t", r)
        return None


def _rename_result(text, r):
    """The statement `text` (without results) defining `r`."""
    return f"{r} = {text.strip()}"


def _clean_attrs(text):
    """An op's text without the barrier attributes of npu-barrier-alloc."""
    t = re.sub(r"\s*\{barrier_gen = \d+ : i64, barrier_group = \d+ : i64\}", "", text)
    return re.sub(r"barrier_gen = \d+ : i64, barrier_group = \d+ : i64,\s*", "", t)


def flatten(text: str, name: str = None) -> Flat:
    """The untiled form of the public function `name` of a post-pipeline
    module (the first function that is not an outlined kernel by default)."""
    funcs = mlir.split_functions(text)
    if name is None:
        cands = [f for f in funcs if "npu.fused_kernel" not in f["header"]]
        if not cands:
            raise NotImplementedError("reader: the module has no function besides its kernels")
        name = cands[-1]["name"]
    f = next(x for x in funcs if x["name"] == name)
    fl = _Flattener(funcs)
    fl.roots = []
    env = {}
    args = []
    for (a, t), txt in zip(f["args"], f["arg_text"]):
        tt = mlir.TType(t.shape, t.elem) if t.shaped else t
        args.append((a, tt))
        fl.types[a] = tt
        if txt.startswith("memref<"):
            env[a] = ("b", fl.new_root(tt, a))
        else:
            env[a] = ("t", a)
    rets = fl.block(parse_block(f["body"]), env) or []
    out_names = []
    for k in rets:
        out_names.append(k[1] if k[0] == "t" else fl.version(k[1]))
    ret = mlir.MOp("func.return", [], [], operands=out_names, text="return")
    fl.ops.append(ret)
    fl.group_of.append(None)
    types = dict(fl.types)
    mf = mlir.MFunc(name, args, [types[v] for v in out_names], fl.ops, types,
                    target=mlir.parse_target(text))
    return Flat(mf, fl.group_of, fl.calls)


def flatten_function_text(text: str, name: str) -> mlir.MFunc:
    return flatten(text, name).func


def groups_of(flat: Flat) -> dict:
    """kernel name -> indices of the untiled ops that came from it."""
    out = {}
    for i, g in enumerate(flat.group_of):
        if g is not None and flat.func.ops[i].name.startswith("linalg."):
            out.setdefault(g, []).append(i)
    return out


def lower_module(text: str, target=None):
    """A post-pipeline module -> lower.Program whose launches run its
    outlined kernels, one launch per kernel's loop nest (several kernels
    chained through a pad, as the int8 and inverted residual chains, one
    launch of their '+'-joined names).  The module's own groups are the
    groups launched; the f16 -> f32 rule of the reference harness applies."""
    from . import lower
    fl = flatten(lower.harness_f32(text))
    prog = lower.lower(fl.func, target, groups=_module_groups(fl) if fl.calls else None)
    return prog, fl


def _module_groups(fl: Flat):
    """The module's outlined kernels as groups of the untiled function:
    {name, ops, inputs (external inputs in first-use order), outputs}."""
    f = fl.func
    by = groups_of(fl)
    for i, g in enumerate(fl.group_of):  # fills of a kernel too
        if g is not None and f.ops[i].name == "linalg.fill" and i not in by.get(g, []):
            by.setdefault(g, []).append(i)
    out = []
    for name in fl.calls:
        ops = sorted(by.get(name, []))
        if not ops:
            continue
        produced = {r for i in ops for r in f.ops[i].results}
        ins, outs = [], []
        for i in ops:
            for v in f.ops[i].all_operands:
                if v not in produced and v not in ins:
                    ins.append(v)
        users = {}
        for j, o in enumerate(f.ops):
            for v in o.all_operands:
                users.setdefault(v, set()).add(j)
        for i in ops:
            for r in f.ops[i].results:
                if users.get(r, set()) - set(ops) and r not in outs:
                    outs.append(r)
        last = f.ops[ops[-1]].results[0]
        if last not in outs:
            outs.append(last)
        out.append({"name": name, "ops": ops, "inputs": ins, "outputs": outs})
    return out
