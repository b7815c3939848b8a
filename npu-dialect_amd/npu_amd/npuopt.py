"""npu-opt, MLIR-free: the reference's pass flags and options over linalg text.

The reference's driver (tools/npu-opt/npu-opt.cpp:33-67) registers the npu
passes with MlirOptMain, so a user writes

    npu-opt in.mlir --npu-fusion --npu-outline-fused-groups \\
        --npu-spatial-tiling=num-cores=256 --npu-temporal-tiling=sram-size=163840 \\
        --npu-bufferize --npu-sram-allocation=sram-size=163840 \\
        --npu-barrier-alloc=barrier-pool-size=4 --npu-cost-evaluate
    npu-opt in.mlir --npu-pipeline

(option names and defaults: include/npu/Transforms/Passes.td:59-73, 79-95,
155-190, 119-149; the pipeline: lib/Transforms/Pipeline.cpp:11-38).  This
module accepts the same flags (``python -m npu_amd.npuopt``) and prints the
module the passes produce, with the decisions of the MLIR-free restatement
(libnpu_host.so: fusion groups, tile-and-fuse, outlining, spatial and
temporal tiles, SRAM plan, barrier allocation, COST_JSON):

* npu-fusion: a (matmul/conv, generic) pair of a fusion group whose
  consumer's best tile config has more than one tile becomes one scf.for
  over the consumer's tiles, the producer chain (its fill, the matmul or
  conv) computed on each tile's slices (FusionPass.cpp:306-359);
* npu-outline-fused-groups: each group becomes
  ``func.func private @fused_<ops>_<idx>(ext inputs) -> (ext outputs)
  attributes {npu.fused_kernel}`` and a ``func.call`` where its last op was
  (OutlineFusedGroupsPass.cpp:205-316); inside a tile-and-fuse loop the call
  takes the tile's slices;
* npu-spatial-tiling: every matmul / batch_matmul / conv_2d_nchw_fchw /
  transpose / generic not inside a loop is tiled on the split dimension the
  cost model picks, ceil(dim / num-cores) per core, remainder peeled
  (SpatialTilingPass.cpp:38-168);
* npu-core-mapping: core_id = (iv - lb) / step, tagged npu.core_id, at the
  head of every outermost loop (CoreMappingPass.cpp:33-73);
* npu-temporal-tiling: every op of those kinds, inside loops or not, tiled by
  the spec-driven search at its own (slice) shape, remainders peeled
  (TemporalTilingPass.cpp:260-336);
* npu-bufferize: tensors become memrefs (slices become subviews, destinations
  are written in place), and every memref defined outside a loop and used in
  it gets an npu.alloc_sram + npu.dma_copy dram_to_sram at the loop's head
  and, when a linalg op writes it, an npu.dma_copy sram_to_dram before the
  loop's end (BufferizePass.cpp:97-222);
* npu-sram-allocation: the dual-end plan of each function's npu.alloc_sram
  buffers (inputs low, outputs high, intermediates in the middle, ping/pong
  for inputs inside loops, weight prefetch into what is left, spills to
  memref.alloc): ``offset``, ``sram_offset_pong``, ``double_buffered``,
  ``prefetch_addr`` (SRAMAllocationPass.cpp:172-363);
* npu-barrier-alloc: ``barrier_group`` / ``barrier_gen`` on every DMA and
  linalg op of a function (DMASchedulingPass.cpp:87-156);
* npu-cost-evaluate: one ``COST_JSON:`` line per function on stderr
  (CostEvaluatePass.cpp:135-158).

Canonicalize and CSE run where the pipeline runs them: full-size slices are
folded away and single-trip loops inlined.  The loop nests follow upstream's
tileUsingSCF + peelForLoopAndSimplifyBounds (a loop over the full tiles, then
the remainder tile as straight-line code, every shape static); the printed
form is this module's, not a byte-for-byte copy of upstream MLIR's printer.
Generic-generic elementwise fusion (upstream linalg::fuseElementwiseOps) is
not restated: a pair of generics stays two ops of the group.

``npu_amd.reader`` reads such modules back and runs each outlined group's
loop nest as one entry-point launch.
"""
from __future__ import annotations

import copy
import re
import sys

from . import host, mlir

PASS_ORDER = ("npu-fusion", "npu-outline-fused-groups", "npu-spatial-tiling",
              "npu-core-mapping", "npu-temporal-tiling", "canonicalize", "cse", "npu-bufferize",
              "npu-sram-allocation", "npu-barrier-alloc", "npu-cost-evaluate")
# Passes.td defaults
OPTIONS = {"npu-spatial-tiling": {"num-cores": 6},
           "npu-temporal-tiling": {"sram-size": 2097152},
           "npu-sram-allocation": {"sram-size": 2097152},
           "npu-barrier-alloc": {"barrier-pool-size": 4}}
TILED_KINDS = ("linalg.matmul", "linalg.batch_matmul", "linalg.conv_2d_nchw_fchw",
               "linalg.transpose", "linalg.generic")
MATRIX = ("linalg.matmul", "linalg.batch_matmul", "linalg.conv_2d_nchw_fchw",
          "linalg.conv_2d_nhwc_fhwc", "linalg.depthwise_conv_2d_nhwc_hwc")


def parse_args(argv):
    """The npu-opt command line -> (input path, {pass: {option: value}} in
    pipeline order, output path).  Options are MLIR's pass-option syntax:
    ``--pass=opt=v`` or ``--pass="opt1=v1 opt2=v2"``."""
    path, out, passes = None, None, {}
    it = iter(argv)
    for a in it:
        if a == "-o":
            out = next(it)
            continue
        if not a.startswith("-") or a == "-":
            if path is not None:
                raise SystemExit(f"npu-opt: a second input file {a}")
            path = a
            continue
        name, _, opts = a.lstrip("-").partition("=")
        if name == "npu-pipeline":
            if opts:
                raise SystemExit("npu-opt: npu-pipeline takes no options")
            for p in PASS_ORDER:
                passes[p] = dict(OPTIONS.get(p, {}))
            continue
        if name not in PASS_ORDER:
            raise SystemExit(f"npu-opt: unknown pass or flag --{name}")
        vals = dict(OPTIONS.get(name, {}))
        for kv in opts.strip("\"'").split():
            k, _, v = kv.partition("=")
            if k not in vals:
                raise SystemExit(f"npu-opt: --{name} has no option '{k}'")
            vals[k] = int(v)
        passes[name] = vals
    order = [p for p in argv if p.startswith("--")]
    given = [p.lstrip("-").partition("=")[0] for p in order
             if p.lstrip("-").partition("=")[0] in PASS_ORDER]
    if given != sorted(given, key=PASS_ORDER.index):
        raise SystemExit("npu-opt: passes run in the pipeline's order "
                         f"({' -> '.join(PASS_ORDER)})")
    return path, passes, out


# ------------------------------------------------------------------ affine maps of the ops
def _lin(expr, names=None):
    """An affine expression (dim index, or text such as 'd2 * 2 + d5') as
    ({dim: coef}, const)."""
    if isinstance(expr, int):
        return {expr: 1}, 0
    terms, const = {}, 0
    for t in expr.replace("-", "+-").split("+"):
        t = t.strip()
        if not t:
            continue
        neg = t.startswith("-")
        t = t.lstrip("-").strip()
        f = [x.strip() for x in t.split("*")]
        coef, dim = (-1 if neg else 1), None
        for x in f:
            m = re.fullmatch(r"d(\d+)", x)
            if m:
                dim = int(m.group(1))
            elif names and x in names:
                dim = names.index(x)
            else:
                coef *= int(x)
        if dim is None:
            const += coef
        else:
            terms[dim] = terms.get(dim, 0) + coef
    return terms, const


def op_maps(op, types):
    """(iteration extents, iterator kinds, [operand map] for ins then outs);
    an operand map is a list of ({dim: coef}, const) per operand dimension,
    None for a scalar operand."""
    sh = lambda v: types[v].shape
    n = op.name
    st = op.attrs.get("strides", [1, 1])
    dl = [1, 1]
    m = re.search(r"dilations\s*=\s*dense<(\[[^\]]*\]|\d+)>", op.text)
    if m:
        v = m.group(1)
        dl = [int(x) for x in v.strip("[]").split(",")] if v.startswith("[") else [int(v)] * 2
    D = lambda *ds: [({d: 1}, 0) for d in ds]
    if n == "linalg.matmul":
        (M, K), (_, N) = sh(op.ins[0]), sh(op.ins[1])
        return [M, N, K], "ppr", [D(0, 2), D(2, 1), D(0, 1)]
    if n == "linalg.batch_matmul":
        (B, M, K), (_, _, N) = sh(op.ins[0]), sh(op.ins[1])
        return [B, M, N, K], "pppr", [D(0, 1, 3), D(0, 3, 2), D(0, 1, 2)]
    if n == "linalg.conv_2d_nchw_fchw":
        N, F, Ho, Wo = sh(op.outs[0])
        _, C, KH, KW = sh(op.ins[1])
        img = [({0: 1}, 0), ({4: 1}, 0), ({2: st[0], 5: dl[0]}, 0), ({3: st[1], 6: dl[1]}, 0)]
        return [N, F, Ho, Wo, C, KH, KW], "pppprrr", [img, D(1, 4, 5, 6), D(0, 1, 2, 3)]
    if n == "linalg.conv_2d_nhwc_fhwc":
        N, Ho, Wo, F = sh(op.outs[0])
        _, KH, KW, C = sh(op.ins[1])
        img = [({0: 1}, 0), ({1: st[0], 4: dl[0]}, 0), ({2: st[1], 5: dl[1]}, 0), ({6: 1}, 0)]
        return [N, Ho, Wo, F, KH, KW, C], "pppprrr", [img, D(3, 4, 5, 6), D(0, 1, 2, 3)]
    if n == "linalg.depthwise_conv_2d_nhwc_hwc":
        N, Ho, Wo, C = sh(op.outs[0])
        KH, KW, _ = sh(op.ins[1])
        img = [({0: 1}, 0), ({1: st[0], 4: dl[0]}, 0), ({2: st[1], 5: dl[1]}, 0), ({3: 1}, 0)]
        return [N, Ho, Wo, C, KH, KW], "pppprr", [img, D(4, 5, 3), D(0, 1, 2, 3)]
    if n == "linalg.fill":
        out = sh(op.outs[0])
        return list(out), "p" * len(out), [None, D(*range(len(out)))]
    if n == "linalg.transpose":
        out = sh(op.outs[0])
        perm = op.attrs["permutation"]
        inv = [perm.index(j) for j in range(len(perm))]
        return list(out), "p" * len(out), [D(*inv), D(*range(len(out)))]
    if n == "linalg.generic":
        maps = op.attrs["maps"]
        its = "".join("p" if i == "parallel" else "r" for i in op.iterators)
        ext = [None] * len(its)
        lin = []
        for v, mp in zip(op.ins + op.outs, maps):
            t = types[v]
            if not t.shaped:
                lin.append(None)
                continue
            row = [_lin(e) for e in mp]
            for (terms, c), size in zip(row, t.shape):
                if len(terms) == 1 and c == 0 and list(terms.values())[0] == 1:
                    ext[list(terms)[0]] = size
            lin.append(row)
        if any(e is None for e in ext):
            raise NotImplementedError(f"{op.results[0]}: a loop of the generic has no extent")
        return ext, its, lin
    raise NotImplementedError(f"npu-opt: no iteration domain for {n}")


# ------------------------------------------------------------------ the emitted IR
class St:
    """One statement: `text` (a region op's header), the names it defines
    and, for scf.for, its body."""

    def __init__(self, text, defs=(), body=None, kind=""):
        self.text, self.defs, self.body, self.kind = text, list(defs), body, kind
        self.attrs = {}

    def uses(self):
        own = set(self.defs)
        return [u for u in re.findall(r"%[\w]+", self.text) if u not in own]


def _sub(text, old, new):
    return re.sub(re.escape(old) + r"(?![\w])", new, text)


def walk(stmts, fn, depth=0, parent=None):
    for s in stmts:
        fn(s, depth, parent)
        if s.body is not None:
            walk(s.body, fn, depth + 1, s)


class Memref:
    """Shape, element type and strided layout of a buffer value."""

    shaped = True

    def __init__(self, shape, elem, strides=None, offset=0):
        self.shape, self.elem = list(shape), elem
        if strides is None:
            strides, acc = [], 1
            for d in reversed(shape):
                strides.insert(0, acc)
                acc *= d
        self.strides, self.offset = list(strides), offset

    def contiguous(self):
        return self.offset == 0 and self.strides == Memref(self.shape, self.elem).strides

    def __str__(self):
        dims = "x".join(str(d) for d in self.shape)
        base = f"{dims}x{self.elem}" if dims else self.elem
        if self.contiguous():
            return f"memref<{base}>"
        off = "?" if self.offset is None else str(self.offset)
        return f"memref<{base}, strided<[{', '.join(str(s) for s in self.strides)}], offset: {off}>>"


class FuncEmitter:
    """Emits one function's body in tensor or memref form."""

    def __init__(self, types, memref, consts, fold=True):
        self.types = dict(types)      # name -> TType (tensor form) or Memref
        self.memref = memref
        self.fold = fold              # canonicalize: full-size slices folded away
        self.consts = consts          # index constants used (hoisted to the top)
        self.stack = [[]]
        self.n = 0

    # naming and constants
    def fresh(self, base=""):
        self.n += 1
        return f"%{base}{'_' if base else ''}{self.n}" if base else f"%{self.n}"

    def c(self, v):
        self.consts.add(v)
        return f"%c{v}"

    def emit(self, st):
        self.stack[-1].append(st)
        return st

    def ty(self, v):
        t = self.types[v]
        return str(t) if isinstance(t, Memref) else (str(t) if t.shaped else t.elem)

    # slices
    def slice(self, v, row, offs, sizes, ext):
        """The slice of v that iteration tile (offs, sizes) reads through the
        operand map `row`; v itself when that is the whole of it."""
        if row is None:
            return v
        t = self.types[v]
        shape = t.shape
        o_txt, o_int, s_out = [], [], []
        dyn = False
        for (terms, c), full in zip(row, shape):
            size = sum(k * ((sizes.get(d, ext[d])) - 1) for d, k in terms.items()) + 1 \
                if terms else 1
            ivs = {d: offs[d] for d in terms if isinstance(offs.get(d), str)}
            const = c + sum(k * offs.get(d, 0) for d, k in terms.items() if d not in ivs)
            if not ivs:
                o_txt.append(str(const))
                o_int.append(const)
            else:
                dyn = True
                o_int.append(None)
                items = list(ivs.items())
                if len(items) == 1 and terms[items[0][0]] == 1 and const == 0:
                    o_txt.append(items[0][1])
                else:
                    names = [f"d{i}" for i in range(len(items))]
                    ex = " + ".join(f"{nm} * {terms[d]}" if terms[d] != 1 else nm
                                    for nm, (d, _) in zip(names, items))
                    if const:
                        ex += f" + {const}"
                    r = self.fresh()
                    self.emit(St(f"{r} = affine.apply affine_map<({', '.join(names)}) -> ({ex})>"
                                 f"({', '.join(iv for _, iv in items)})", [r], kind="index"))
                    o_txt.append(r)
            s_out.append(size)
        if self.fold and not dyn and all(o == 0 for o in o_int) and s_out == list(shape):
            return v
        r = self.fresh("subview" if self.memref else "extracted_slice")
        ones = ", ".join("1" for _ in shape)
        if self.memref:
            off = None if dyn else t.offset + sum(o * s for o, s in zip(o_int, t.strides)) \
                if t.offset is not None else None
            nt = Memref(s_out, t.elem, t.strides, off)
            if nt.contiguous() and off is None:
                nt.offset = None
            self.types[r] = nt
            self.emit(St(f"{r} = memref.subview {v}[{', '.join(o_txt)}] "
                         f"[{', '.join(map(str, s_out))}] [{ones}] : {t} to {nt}", [r],
                         kind="subview"))
        else:
            nt = mlir.TType(s_out, t.elem)
            self.types[r] = nt
            self.emit(St(f"{r} = tensor.extract_slice {v}[{', '.join(o_txt)}] "
                         f"[{', '.join(map(str, s_out))}] [{ones}] : {t} to {nt}", [r],
                         kind="slice"))
        self.slice_of = getattr(self, "slice_of", {})
        self.slice_of[r] = (v, o_txt, s_out)
        return r

    def insert(self, tile, dest_slice, dest):
        """tensor.insert_slice of a computed tile back into `dest` where
        `dest_slice` was extracted (tensor form)."""
        src, o_txt, s_out = self.slice_of[dest_slice]
        r = self.fresh("inserted_slice")
        self.types[r] = self.types[dest]
        ones = ", ".join("1" for _ in s_out)
        self.emit(St(f"{r} = tensor.insert_slice {tile} into {dest}[{', '.join(o_txt)}] "
                     f"[{', '.join(map(str, s_out))}] [{ones}] : {self.types[tile]} into "
                     f"{self.types[dest]}", [r], kind="insert"))
        return r

    # ops
    def linalg(self, op, ins, outs, result=None):
        """Prints op with operands renamed; returns its result (tensor form)."""
        text = op.text.strip()
        m = re.match(r"^((?:%[\w]+(?::\d+)?\s*,\s*)*%[\w]+(?::\d+)?)\s*=\s*", text)
        if m:
            text = text[m.end():]
        ig = mlir._find_group(text, "ins")
        og = mlir._find_group(text, "outs")
        if ig is not None:
            text = text.replace(f"ins({ig})", f"ins({', '.join(ins)} : "
                                f"{', '.join(self.ty(v) for v in ins)})", 1)
        text = text.replace(f"outs({og})", f"outs({', '.join(outs)} : "
                            f"{', '.join(self.ty(v) for v in outs)})", 1)
        # result types after the last `->` at depth 0 (after the region)
        cut = _result_arrow(text)
        if cut is not None:
            text = text[:cut].rstrip()
        if self.memref:
            self.emit(St(text, [], kind="linalg"))
            return None
        r = result or self.fresh()
        self.types[r] = self.types[outs[0]]
        self.emit(St(f"{r} = {text} -> {self.ty(outs[0])}", [r], kind="linalg"))
        return r

    def loop(self, iv, lb, ub, step, it=None, init=None, res=None):
        hdr = f"scf.for {iv} = {self.c(lb)} to {self.c(ub)} step {self.c(step)}"
        if it:
            hdr = f"{res} = {hdr} iter_args({it} = {init}) -> ({self.ty(init)})"
        st = St(hdr, [res] if res else [], body=[], kind="for")
        st.attrs["ivs"] = [iv] + ([it] if it else [])
        self.emit(st)
        self.stack.append(st.body)
        return st

    def end(self, yielded=None):
        if yielded is not None:
            self.emit(St(f"scf.yield {yielded} : {self.ty(yielded)}", kind="yield"))
        self.stack.pop()


def _result_arrow(text):
    """Index of a trailing `-> type` at depth 0 (a linalg op's result types)."""
    depth, last = 0, None
    i = 0
    while i < len(text):
        ch = text[i]
        if ch in "([{<":
            depth += 1
        elif ch in ")]}>" and not (ch == ">" and text[i - 1] == "-"):
            depth -= 1
        elif depth == 0 and text.startswith("->", i):
            last = i
        i += 1
    return last


# ------------------------------------------------------------------ tiling
class Tiler:
    """Emits `op` tiled over `tiles` ([(iteration dim, tile size)]) with the
    remainder of every loop peeled.  At each tile, `inner(op, ins, outs,
    offs, sizes)` emits the tile's computation (the op on its slices, the op
    tiled again, or a fused chain) and returns its result (tensor form)."""

    def __init__(self, em: FuncEmitter):
        self.em = em

    def run(self, op, ins, out, tiles, inner, types, slice_ins=True):
        em = self.em
        ext, its, maps = op_maps(op, types)
        tiles = [(d, t) for d, t in tiles if 0 < t < ext[d]]

        def rec(k, offs, sizes, acc):
            if k == len(tiles):
                s_ins = [em.slice(v, mp, offs, sizes, ext) for v, mp in zip(ins, maps)] \
                    if slice_ins else list(ins)
                s_out = em.slice(acc, maps[len(op.ins)], offs, sizes, ext)
                r = inner(op, s_ins, [s_out], offs, sizes)
                if em.memref:
                    return acc
                if s_out == acc:
                    return r
                return em.insert(r, s_out, acc)
            d, T = tiles[k]
            nfull, rem = divmod(ext[d], T)
            cur = acc
            if nfull >= 2:
                iv = em.fresh("arg")
                if em.memref:
                    em.loop(iv, 0, nfull * T, T)
                    rec(k + 1, {**offs, d: iv}, {**sizes, d: T}, cur)
                    em.end()
                else:
                    it, res = em.fresh("arg"), em.fresh()
                    em.types[it] = em.types[res] = em.types[cur]
                    em.loop(iv, 0, nfull * T, T, it, cur, res)
                    em.end(rec(k + 1, {**offs, d: iv}, {**sizes, d: T}, it))
                    cur = res
            elif nfull == 1:
                cur = rec(k + 1, {**offs, d: 0}, {**sizes, d: T}, cur)
            if rem:
                cur = rec(k + 1, {**offs, d: nfull * T}, {**sizes, d: rem}, cur)
            return cur

        return rec(0, {}, {}, out)


def bind_types(op, bind, types):
    """types of op's operands under `bind` (names -> current names), keyed by
    op's own operand names."""
    out = dict(types)
    for v in op.ins + op.outs:
        if v in bind:
            t = types[bind[v]]
            out[v] = mlir.TType(t.shape, t.elem) if isinstance(t, Memref) else t
    return out


def _single_op_graph(op, ins, outs, types):
    """A one-op function of op at the shapes of (ins, outs) for the host
    library's per-op decisions."""
    args = []
    for v in ins + outs:
        t = types[v]
        if isinstance(t, Memref):
            t = mlir.TType(t.shape, t.elem)
        args.append((v, t))
    import copy
    o = copy.copy(op)
    o.ins, o.outs = list(ins), list(outs)
    o.results = ["%__r"]
    ot = types[outs[0]]
    o.result_types = [mlir.TType(ot.shape, ot.elem)]
    ty = {n: t for n, t in args}
    ty["%__r"] = o.result_types[0]
    f = mlir.MFunc("one", args, o.result_types, [o], ty)
    return f


# ------------------------------------------------------------------ the driver
def run_passes(text: str, passes: dict):
    """Runs `passes` ({name: options}, pipeline order) on the module text.
    Returns (module text, COST_JSON lines, remarks)."""
    funcs = mlir.parse_functions(text)
    host.spec_reset()  # one npu-opt process per module
    tparams = mlir.parse_target(text)
    t = host.target_from_params(tparams) if tparams else host.default_target()
    on = lambda p: p in passes
    remarks, cost_lines, out_funcs = [], [], []
    for f in funcs:
        out_funcs += _function(f, t, passes, remarks)
    if on("npu-sram-allocation"):
        for fn in out_funcs:
            _sram_allocation(fn, passes["npu-sram-allocation"]["sram-size"], remarks)
    if on("npu-barrier-alloc"):
        for fn in out_funcs:
            _barrier_alloc(fn, passes["npu-barrier-alloc"]["barrier-pool-size"], remarks)
    if on("npu-cost-evaluate"):
        for fn in out_funcs:
            cost_lines.append(_cost(fn, t, remarks))
    body = "\n".join(_print_func(fn) for fn in out_funcs)
    head = ""
    m = re.search(r"module\s+attributes\s*\{.*?\}\s*\{", text, re.S)
    aliases = re.findall(r"^\s*(#[\w.]+\s*=\s*#npu\.target<[^>]*>)", text, re.M)
    if aliases:
        head = "\n".join(aliases) + "\n"
    mod = (m.group(0)[:-1].strip() if m else "module") + " {"
    return f"{head}{mod}\n{body}}}\n", cost_lines, remarks


class OutFunc:
    def __init__(self, name, private, args, rtypes, body, types, consts, attrs=""):
        self.name, self.private, self.args, self.rtypes = name, private, args, rtypes
        self.body, self.types, self.consts, self.attrs = body, types, consts, attrs
        self.source = None  # (MFunc, op indices) the function computes


def _function(f: mlir.MFunc, t, passes, remarks):
    """The function f after fusion/outlining/tiling: [OutFunc] (outlined
    kernels first, then f)."""
    on = lambda p: p in passes
    memref = on("npu-bufferize")
    g = host.Graph(f)
    ops = f.ops
    groups = host.outline_groups(g, t) if on("npu-outline-fused-groups") else []
    grouped = {i: gi for gi, grp in enumerate(groups) for i in grp["ops"]}
    # tile-and-fuse: one loop per (matrix op, generic) pair whose consumer
    # tiles into more than one tile; the chain fill -> anchor -> generic
    fused = {}
    uses = {}
    for o in ops:
        for v in o.all_operands:
            uses[v] = uses.get(v, 0) + 1
    if on("npu-fusion"):
        for grp in host.fusion_groups(g, t):
            for a, b in zip(grp, grp[1:]):
                oa, ob = ops[a], ops[b]
                if oa.name not in MATRIX or ob.name != "linalg.generic":
                    continue
                if not oa.results or oa.results[0] not in ob.ins:
                    continue
                tiled, cost = host.tile_and_fuse(g, t, b)
                if not tiled:
                    continue
                fill = [i for i, o in enumerate(ops) if o.name == "linalg.fill"
                        and o.results and o.results[0] == oa.outs[0]]
                chain = fill + [a, b]
                # the chain computes the consumer's tile from slices: every
                # intermediate has its one use in the chain, and the
                # consumer reads the producer and writes its output through
                # the same map of output coordinates
                _, _, gm = op_maps(ob, f.types)
                k = ob.ins.index(oa.results[0])
                if gm[k] != gm[-1] or any(len(tm) != 1 or c for tm, c in gm[-1]) or \
                        any(uses.get(ops[i].results[0], 0) != 1 for i in chain[:-1]):
                    remarks.append(f"{f.name}: {ob.results[0]} not tiled and fused: its chain "
                                   "does not map the consumer's tile to its producers")
                    continue
                if groups and len({grouped.get(i) for i in chain}) != 1:
                    remarks.append(f"{f.name}: {ob.results[0]} not tiled and fused: its chain "
                                   "spans outlined groups")
                    continue
                if groups and sorted(groups[grouped[b]]["ops"]) != sorted(chain):
                    remarks.append(f"{f.name}: {ob.results[0]} not tiled and fused: its group "
                                   "holds ops outside the fused chain")
                    continue
                fused[b] = (chain, cost.tiles)
    out = []
    consts = set()
    # outlined kernels
    kernel_of = {}
    for gi, grp in enumerate(groups):
        tile = next((v for b, v in fused.items() if b in grp["ops"]), None)
        kernel_of[gi] = grp["name"]
        if tile is None:
            k = _kernel(f, grp, {}, t, passes)
            out.append(k)
    # the parent
    em = FuncEmitter(_arg_types(f, memref), memref, consts, "canonicalize" in passes)
    bind = {}
    emitted_groups = set()
    for i, op in enumerate(ops):
        if op.name == "func.return":
            vals = [bind.get(v, v) for v in op.operands]
            em.emit(St(f"return {', '.join(vals)} : {', '.join(em.ty(v) for v in vals)}"
                       if vals else "return", kind="return"))
            continue
        if i in grouped:
            gi = grouped[i]
            if gi in emitted_groups or i != max(groups[gi]["ops"]):
                continue
            emitted_groups.add(gi)
            grp = groups[gi]
            b = next((b for b in fused if b in grp["ops"]), None)
            if b is not None:
                out.append(_fused(f, fused[b], em, bind, t, passes, grp))
            else:
                _call(em, grp, grp["name"], bind, f)
            continue
        if i in fused:
            _fused(f, fused[i], em, bind, t, passes)
            continue
        if any(i in ch for ch, _ in fused.values()):
            continue
        _plain_op(f, i, em, bind, t, passes, top=True)
    pf = OutFunc(f.name, False, [(n, em.types[n]) for n, _ in f.args],
                 [em.types[v] for v in _returned(em)], em.stack[0], em.types, consts)
    out.append(pf)
    for k in out:
        if on("npu-core-mapping"):
            _core_mapping(k, remarks)
        if memref:
            _dma_insertion(k)
    return out


def _returned(em):
    r = [s for s in em.stack[0] if s.kind == "return"]
    if not r:
        return []
    m = re.match(r"return\s+(.*?)\s*:", r[0].text)
    return [v.strip() for v in m.group(1).split(",")] if m else []


def _arg_types(f, memref):
    ty = {}
    for n, tt in f.args:
        ty[n] = Memref(tt.shape, tt.elem) if memref and tt.shaped else tt
    return ty


def _value_type(t, memref):
    if isinstance(t, Memref) or not memref or not t.shaped:
        return t
    return Memref(t.shape, t.elem)


def _plain_op(f, i, em, bind, t, passes, top):
    """One op of a function body, tiled where the passes tile it."""
    op = f.ops[i]
    on = lambda p: p in passes
    if op.name == "arith.constant":
        em.types[op.results[0]] = op.result_types[0]
        em.emit(St(op.text.strip(), op.results, kind="const"))
        return
    if op.name == "tensor.empty":
        r = op.results[0]
        if em.memref:
            em.types[r] = Memref(op.result_types[0].shape, op.result_types[0].elem)
            em.emit(St(f"{r} = memref.alloc() {{alignment = 64 : i64}} : {em.types[r]}", [r],
                       kind="alloc"))
        else:
            em.types[r] = op.result_types[0]
            em.emit(St(op.text.strip(), [r], kind="empty"))
        return
    if not op.name.startswith("linalg."):
        # tensor.pad, reshapes: kept whole (in memref form, as a tensor round trip)
        text = op.text.strip()
        for v in op.all_operands:
            if v in bind:
                text = _sub(text, v, bind[v])
        if em.memref and op.results:
            return _tensor_op_in_memref(op, em, bind, text)
        for r, rt in zip(op.results, op.result_types):
            em.types[r] = rt
        em.emit(St(text, op.results, kind="other"))
        return
    _tiled_linalg(op, bind, em, t, passes, top)


def _tensor_op_in_memref(op, em, bind, text):
    """A non-linalg tensor op (tensor.pad, reshape) in memref form: its
    operands as tensors (bufferization.to_tensor), its result copied into a
    new buffer."""
    for v in op.all_operands:
        b = bind.get(v, v)
        if isinstance(em.types.get(b), Memref):
            tv = em.fresh()
            tt = em.types[b]
            em.types[tv] = mlir.TType(tt.shape, tt.elem)
            em.emit(St(f"{tv} = bufferization.to_tensor {b} : {tt} to {em.types[tv]}", [tv],
                       kind="to_tensor"))
            text = _sub(text, b, tv)
    r = op.results[0]
    tr = em.fresh()
    em.emit(St(_sub(text, r, tr), [tr], kind="other"))
    rt = op.result_types[0]
    em.types[tr] = rt
    em.types[r] = Memref(rt.shape, rt.elem)
    em.emit(St(f"{r} = bufferization.to_buffer {tr} : {rt} to {em.types[r]}", [r],
               kind="to_buffer"))


def _temporal_then(em, t, passes):
    """The tile callback that applies npu-temporal-tiling to a tile's op (or
    to a whole op outside any loop) where the spec-driven search at the
    op's own shape gives more than one tile, and prints the op otherwise."""

    def temporal(o, i_, o_, offs=None, sizes=None):
        if "npu-temporal-tiling" in passes and o.name in TILED_KINDS:
            sf = _single_op_graph(o, i_, o_, em.types)
            tgt = _with_sram(t, passes["npu-temporal-tiling"]["sram-size"])
            ts, cost = host.temporal(host.Graph(sf), tgt, 0)
            if ts and cost.num_tiles > 1:
                leaf = lambda o2, a, b, *_: em.linalg(o2, a, b)
                return Tiler(em).run(sf.ops[0], list(i_), o_[0], list(enumerate(ts)), leaf,
                                     sf.types)
        return em.linalg(o, i_, o_)

    return temporal


def _tiled_linalg(op, bind, em, t, passes, top):
    """A linalg op: npu-spatial-tiling when it is outside any loop, then
    npu-temporal-tiling of each tile, where the passes and the decisions tile
    it (SpatialTilingPass.cpp:38-168, TemporalTilingPass.cpp:260-336)."""
    ins = [bind.get(v, v) for v in op.ins]
    out = bind.get(op.outs[0], op.outs[0])
    o = copy.copy(op)
    o.ins, o.outs = ins, [out]
    temporal = _temporal_then(em, t, passes)
    if top and "npu-spatial-tiling" in passes and op.name in TILED_KINDS:
        sf = _single_op_graph(o, ins, [out], em.types)
        d = host.spatial(host.Graph(sf), t, 0, passes["npu-spatial-tiling"]["num-cores"])
        if d is not None:
            r = Tiler(em).run(o, ins, out, [(d.iter_dim, d.tile_size)], temporal, sf.types)
            return _bind_result(op, r, out, em, bind)
    return _bind_result(op, temporal(o, ins, [out]), out, em, bind)


def _bind_result(op, r, out, em, bind):
    bind[op.results[0]] = out if em.memref else r
    return bind[op.results[0]]


def _with_sram(t, sram):
    t2 = copy.copy(t)
    t2.sram_per_core = sram
    return t2


def _kernel(f, grp, shapes, t, passes):
    """The outlined function of group `grp` (OutlineFusedGroupsPass.cpp:205-303):
    arguments = the group's external inputs in first-use order, results =
    its external outputs; `shapes` gives the inputs' slice types when a
    tile-and-fuse loop calls the kernel once per tile."""
    memref = "npu-bufferize" in passes
    args, ty, bind = [], {}, {}
    for k, v in enumerate(grp["inputs"]):
        a = f"%arg{k}"
        ty[a] = _value_type(shapes.get(v, f.types[v]), memref)
        args.append((a, ty[a]))
        bind[v] = a
    em = FuncEmitter(ty, memref, set(), "canonicalize" in passes)
    for i in grp["ops"]:
        _plain_op(f, i, em, bind, t, passes, top=True)
    rets = [bind.get(v, v) for v in grp["outputs"]]
    em.emit(St(f"return {', '.join(rets)} : {', '.join(em.ty(v) for v in rets)}", kind="return"))
    k = OutFunc(grp["name"], True, args, [em.types[v] for v in rets], em.stack[0], em.types,
                em.consts, attrs="npu.fused_kernel")
    return k


def _call(em, grp, name, bind, f, args=None, out_types=None):
    """func.call of an outlined group where its last op was."""
    vals = args or [bind.get(v, v) for v in grp["inputs"]]
    outs = grp["outputs"]
    r = em.fresh()
    rtypes = [_value_type((out_types or f.types)[v], em.memref) for v in outs]
    names = [r] if len(outs) == 1 else [f"{r}#{k}" for k in range(len(outs))]
    lhs = r if len(outs) == 1 else f"{r}:{len(outs)}"
    for v, n, tt in zip(outs, names, rtypes):
        bind[v] = n
        em.types[n] = tt
    sig = f"({', '.join(em.ty(v) for v in vals)}) -> " + \
          (str(rtypes[0]) if len(rtypes) == 1 else f"({', '.join(map(str, rtypes))})")
    em.emit(St(f"{lhs} = func.call @{name}({', '.join(vals)}) : {sig}", [r], kind="call"))
    return names


def _user_tile(user, gen, offs, sizes, types):
    """The iteration tile of `user`, an op of a fused chain, that writes or
    reads the consumer's output tile (offs, sizes): the chain's ops share
    the consumer's output coordinates; their reduction loops stay whole."""
    if user is gen:
        return offs, sizes
    _, _, gm = op_maps(gen, types)
    _, _, um = op_maps(user, types)
    o2, s2 = {}, {}
    for (gt, _), (ut, _) in zip(gm[-1], um[-1]):
        gd, ud = list(gt)[0], list(ut)[0]
        if gd in offs:
            o2[ud] = offs[gd]
        if gd in sizes:
            s2[ud] = sizes[gd]
    return o2, s2


def _fused(f, fuse, em, bind, t, passes, grp=None):
    """The tile-and-fuse loop over the consumer generic's tiles
    (FusionPass.cpp:306-359).  With outlining (`grp`), each tile calls the
    outlined kernel on the slices of the group's inputs (the kernel, typed
    at the first tile's slices, is returned); without, the chain's ops run
    on the slices inside the loop."""
    chain, tiles = fuse
    gen = f.ops[chain[-1]]
    kernel = {}

    def slice_for(o, v, k, offs, sizes):
        uo, us = _user_tile(o, gen, offs, sizes, f.types)
        uext, _, um = op_maps(o, f.types)
        return em.slice(bind.get(v, v), um[k], uo, us, uext)

    def call_kernel(op, s_ins, s_outs, offs, sizes):
        args, shapes = [], {}
        for v in grp["inputs"]:
            if v == gen.outs[0]:
                s = s_outs[0]
            else:
                o = next(f.ops[i] for i in chain if v in f.ops[i].ins + f.ops[i].outs)
                s = slice_for(o, v, (o.ins + o.outs).index(v), offs, sizes)
            args.append(s)
            shapes[v] = em.types[s]
        if not kernel:
            kernel["k"] = _kernel(f, grp, shapes, t, passes)
        tt = em.types[s_outs[0]]
        out_types = {v: mlir.TType(tt.shape, tt.elem) for v in grp["outputs"]}
        return _call(em, grp, grp["name"], {}, f, args=args, out_types=out_types)[0]

    def chain_ops(op, s_ins, s_outs, offs, sizes):
        local = {}
        for i in chain:
            o = f.ops[i]
            ins_ = [local[v] if v in local else slice_for(o, v, k, offs, sizes)
                    for k, v in enumerate(o.ins)]
            ov = o.outs[0]
            outs_ = s_outs if o is gen else \
                [local[ov] if ov in local else slice_for(o, ov, len(o.ins), offs, sizes)]
            r = em.linalg(o, ins_, outs_)
            local[o.results[0]] = r if r is not None else outs_[0]
        return local[gen.results[0]]

    ins = [bind.get(v, v) for v in gen.ins]
    out = bind.get(gen.outs[0], gen.outs[0])
    r = Tiler(em).run(gen, ins, out, list(enumerate(tiles)),
                      call_kernel if grp else chain_ops, f.types, slice_ins=False)
    bind[gen.results[0]] = out if em.memref else r
    return kernel.get("k")


# ------------------------------------------------------------------ later passes
def _core_mapping(fn: OutFunc, remarks):
    """core_id = (iv - lb) / step at the head of every outermost loop."""
    for s in fn.body:
        if s.kind != "for":
            continue
        m = re.match(r"(?:%[\w]+\s*=\s*)?scf\.for\s+(%[\w]+)\s*=\s*%c(\d+)\s+to\s+%c\d+\s+step\s+%c(\d+)",
                     s.text)
        if not m:
            continue
        iv, lb, step = m.group(1), int(m.group(2)), int(m.group(3))
        base = iv.lstrip("%")
        a, b, c = f"%{base}_off", f"%{base}_core", f"%{base}_core_id"
        fn.consts.update([lb, step])
        s.body[0:0] = [St(f"{a} = arith.subi {iv}, %c{lb} : index", [a], kind="index"),
                       St(f"{b} = arith.divui {a}, %c{step} : index", [b], kind="index"),
                       St(f"{c} = arith.index_cast {b} {{npu.core_id}} : index to i64", [c],
                          kind="index")]
        remarks.append(f"{fn.name}: core mapping: loop mapped to cores")


def _dma_insertion(fn: OutFunc):
    """npu-bufferize's phase 3 (BufferizePass.cpp:97-222) on every loop,
    outermost first."""
    defs = {}

    def collect(s, depth, parent):
        for d in s.defs:
            defs[d] = s

    walk(fn.body, collect)
    counter = [0]

    def process(stmts):
        for s in stmts:
            if s.kind != "for":
                continue
            inside = set()
            walk(s.body, lambda x, d, p: inside.update(x.defs))
            inside.update(s.attrs.get("ivs", []))
            inputs, outputs = [], set()

            def scan(x, depth, parent):
                if x.kind == "yield":
                    return
                outs = []
                if x.kind == "linalg":
                    og = mlir._find_group(x.text, "outs")
                    outs = re.findall(r"%[\w]+", og.split(":")[0]) if og else []
                for u in x.uses():
                    if u in inside or u not in defs:
                        continue
                    dk = defs[u].kind
                    if dk in ("sram", "dma", "const", "index") or \
                            not isinstance(fn.types.get(u), Memref):
                        continue
                    if u not in inputs:
                        inputs.append(u)
                    if u in outs:
                        outputs.add(u)

            walk(s.body, scan)
            if inputs:
                head, tail, ren = [], [], {}
                for u in inputs:
                    counter[0] += 1
                    sb = f"%sram_{counter[0]}"
                    ren[u] = sb
                    fn.types[sb] = fn.types[u]
                    st = St(f"{sb} = npu.alloc_sram : {fn.types[u]}", [sb], kind="sram")
                    defs[sb] = st
                    head.append(st)
                    head.append(St(f"npu.dma_copy {u} to {sb} dir dram_to_sram : {fn.types[u]} to "
                                   f"{fn.types[u]}", kind="dma"))
                for u in inputs:
                    if u in outputs:
                        tail.append(St(f"npu.dma_copy {ren[u]} to {u} dir sram_to_dram : "
                                       f"{fn.types[u]} to {fn.types[u]}", kind="dma"))

                def rename(x, depth, parent):
                    for u, sb in ren.items():
                        x.text = _sub(x.text, u, sb)

                walk(s.body, rename)
                s.body[0:0] = head
                if tail:
                    y = [i for i, x in enumerate(s.body) if x.kind == "yield"]
                    at = y[0] if y else len(s.body)
                    s.body[at:at] = tail
            process(s.body)

    process(fn.body)


def _sram_allocation(fn: OutFunc, sram, remarks):
    """Plans the function's npu.alloc_sram buffers with the dual-end
    allocator and sets their attributes."""
    allocs, step, pos, users = [], [0], {}, {}

    def number(s, depth, parent):
        pos[id(s)] = step[0]
        step[0] += 1
        if s.kind == "sram":
            allocs.append((s, depth > 0))
        for u in s.uses():
            users.setdefault(u, []).append(s)

    walk(fn.body, number)
    if not allocs:
        return
    bufs = []
    for s, in_loop in allocs:
        b = s.defs[0]
        d2s = any(re.search(r"dir dram_to_sram", x.text) and
                  re.search(r"to\s+" + re.escape(b) + r"(?![\w])", x.text) for x in users.get(b, []))
        s2d = any(re.search(r"dir sram_to_dram", x.text) and
                  re.match(r"npu\.dma_copy\s+" + re.escape(b) + r"(?![\w])", x.text)
                  for x in users.get(b, []))
        role = 1 if s2d else (0 if d2s else 2)
        t = fn.types[b]
        nbytes = 1
        for d in t.shape:
            nbytes *= d
        nbytes *= max(1, mlir.TYPE_BITS.get(t.elem, 32) // 8)
        us = [pos[id(x)] for x in users.get(b, [])] + [pos[id(s)]]
        sb = host.SramBuffer(value=len(bufs), role=role, bytes=nbytes, first_use=min(us),
                             last_use=max(us), in_loop=int(in_loop))
        bufs.append(sb)
    summ = host.sram_allocation(bufs, sram)
    for (s, _), b in zip(allocs, bufs):
        name = s.defs[0]
        if b.spilled:
            s.text = f"{name} = memref.alloc() : {fn.types[name]}"
            s.kind = "alloc"
            continue
        attrs = []
        if b.double_buffered:
            attrs += [f"sram_offset_pong = {b.addr_pong} : i64", "double_buffered"]
        if b.prefetch_addr >= 0:
            attrs.append(f"prefetch_addr = {b.prefetch_addr} : i64")
        a = f" {{{', '.join(attrs)}}}" if attrs else ""
        s.text = f"{name} = npu.alloc_sram offset {b.addr}{a} : {fn.types[name]}"
    if summ.spilled:
        remarks.append(f"{fn.name}: SRAM allocation: {summ.spilled} buffer(s) spilled to DDR")
    if summ.prefetched:
        remarks.append(f"{fn.name}: Weight prefetch: {summ.prefetched} buffer(s) prefetched")


def _barrier_alloc(fn: OutFunc, pool, remarks):
    ops = []

    def cls(s, depth, parent):
        if s.kind == "dma":
            ops.append((s, "dma_in" if "dram_to_sram" in s.text else "dma_out"))
        elif s.kind == "linalg":
            ops.append((s, "compute"))

    walk(fn.body, cls)
    if not ops:
        return
    res = host.barrier_alloc([k for _, k in ops], pool)
    for (s, _), (sg, bid, gen) in zip(ops, res):
        attr = f"barrier_gen = {gen} : i64, barrier_group = {bid} : i64"
        s.text = _add_attrs(s.text, attr)
    n_sub = max(r[0] for r in res) + 1
    n_gen = max(r[2] for r in res) + 1
    remarks.append(f"{fn.name}: barrier alloc: {n_sub} subgraphs, {pool} barriers, {n_gen} "
                   f"generation(s){' (double-buffered)' if n_gen > 1 else ''}")


def _add_attrs(text, attr):
    if text.startswith("npu.dma_copy"):
        i = text.index(" : ")
        return f"{text[:i]} {{{attr}}}{text[i:]}"
    # linalg op in memref form: attributes go in the attr-dict after the op name
    m = re.match(r"(linalg\.[\w]+)(\s*\{)", text)
    if m:
        return f"{m.group(1)} {{{attr}, " + text[m.end():].lstrip()
    m = re.match(r"(linalg\.[\w]+)", text)
    return f"{m.group(1)} {{{attr}}}" + text[m.end():]


def _tensor_bytes(t):
    n = 1
    for d in t.shape:
        n *= d
    return n * max(1, mlir.TYPE_BITS.get(t.elem, 32) // 8)


def _cost(fn: OutFunc, t, remarks):
    """The function's COST_JSON record, computed from the IR as it stands the
    way CostEvaluatePass.cpp:57-168 does: the roofline of its linalg ops (the
    tile ops present in the IR, external operands counted once each), DMA
    bytes by direction from each dma_copy's source type, matrix / DSP
    cycles, peak SRAM (offset + bytes of each npu.alloc_sram), and the
    largest trip-count product of an outermost loop nest."""
    insts, dma = [], {"in": 0, "out": 0}
    peak = [0]
    trips = [0]

    def collect(s, depth, parent):
        if s.kind == "linalg":
            insts.append(s)
        elif s.kind == "dma":
            src = mlir.parse_type(s.text.rsplit(":", 1)[1].split(" to ")[0])
            dma["in" if "dram_to_sram" in s.text else "out"] += _tensor_bytes(src)
        elif s.kind == "sram":
            m = re.search(r"offset\s+(\d+)", s.text.split(":")[0])
            off = int(m.group(1)) if m else 0
            peak[0] = max(peak[0], off + _tensor_bytes(fn.types[s.defs[0]]))

    walk(fn.body, collect)

    def trip(s):
        m = re.search(r"%c(\d+)\s+to\s+%c(\d+)\s+step\s+%c(\d+)", s.text)
        lb, ub, st = map(int, m.groups())
        return max(0, -(-(ub - lb) // st))

    for s in fn.body:
        if s.kind == "for":
            prod = [trip(s)]
            walk(s.body, lambda x, d, p: prod.append(trip(x)) if x.kind == "for" else None)
            total = 1
            for v in prod:
                total *= v
            trips[0] = max(trips[0], total)
    ops, types, args = [], {}, []
    produced = set()
    for s in insts:
        op = mlir.parse_op(s.text)
        for v, ty in zip(op.ins + op.outs, op.attrs["in_types"] + op.attrs["out_types"]):
            if v not in types and v not in produced:
                types[v] = ty
                args.append((v, ty))
        for r, ty in zip(op.results, op.result_types):
            types[r] = ty
            produced.add(r)
        ops.append(op)
    kc = host.KernelCost()
    kc.num_linalg_ops = len(ops)
    if ops:
        g = host.Graph(mlir.MFunc(fn.name, args, [], ops, types))
        cm = host.CostModel(g, t)
        rl = cm.roofline(list(range(len(ops))))
        kc.flops, kc.mem_bytes = rl.flops, rl.mem_bytes
        kc.arithmetic_intensity, kc.time_sec = rl.arithmetic_intensity, rl.time_sec
        kc.memory_bound, kc.efficiency = rl.is_memory_bound, rl.efficiency
        for k, op in enumerate(ops):
            cyc = cm.compute_cycles(k)
            if op.name in ("linalg.matmul", "linalg.batch_matmul", "linalg.conv_2d_nchw_fchw"):
                kc.matrix_cycles += cyc
            else:
                kc.dsp_cycles += cyc
    kc.dma_in_bytes, kc.dma_out_bytes = dma["in"], dma["out"]
    kc.peak_sram_bytes = peak[0]
    kc.num_tile_iterations = trips[0]
    kc.sram_budget = t.sram_per_core
    remarks.append(f"{fn.name}: roofline: {kc.flops:.2e} FLOP, {kc.mem_bytes:.2e} bytes, "
                   f"AI={kc.arithmetic_intensity:.1f} FLOP/B, "
                   f"{'MEM-bound' if kc.memory_bound else 'COMPUTE-bound'}, "
                   f"eff={kc.efficiency * 100:.1f}%")
    return host.cost_json(fn.name, kc)


def _print_func(fn: OutFunc) -> str:
    args = ", ".join(f"{n}: {t}" for n, t in fn.args)
    res = ""
    if fn.rtypes:
        res = " -> " + (str(fn.rtypes[0]) if len(fn.rtypes) == 1
                        else "(" + ", ".join(map(str, fn.rtypes)) + ")")
    vis = "private " if fn.private else ""
    attrs = f" attributes {{{fn.attrs}}}" if fn.attrs else ""
    lines = [f"  func.func {vis}@{fn.name}({args}){res}{attrs} {{"]
    for v in sorted(fn.consts):
        lines.append(f"    %c{v} = arith.constant {v} : index")

    def emit(stmts, ind):
        for s in stmts:
            if s.body is not None:
                lines.append(" " * ind + s.text + " {")
                emit(s.body, ind + 2)
                lines.append(" " * ind + "}")
            else:
                for k, ln in enumerate(s.text.split("\n")):
                    lines.append((" " * ind if k == 0 else "") + ln)

    emit(fn.body, 4)
    lines.append("  }")
    return "\n".join(lines) + "\n"


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    path, passes, out = parse_args(argv)
    text = sys.stdin.read() if path in (None, "-") else open(path).read()
    mod, costs, remarks = run_passes(text, passes)
    for r in remarks:
        print(f"remark: {r}", file=sys.stderr)
    for c in costs:
        print(c, file=sys.stderr)
    if out:
        with open(out, "w") as fh:
            fh.write(mod)
    else:
        sys.stdout.write(mod)
    return 0


if __name__ == "__main__":
    sys.exit(main())
