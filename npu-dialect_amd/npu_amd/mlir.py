"""Reads the tensor-level linalg subset NPU-Dialect compiles into a flat op list.

The reference's inputs are `func.func` bodies of `arith.constant`,
`tensor.empty`, `tensor.pad`, `linalg.fill`, `linalg.matmul`,
`linalg.batch_matmul`, `linalg.conv_2d_nchw_fchw`, `linalg.generic` (ReLU /
add bodies) and `func.return` (SURVEY of test/**/*.mlir); the configurations
here add `linalg.conv_2d_nhwc_fhwc`, `linalg.depthwise_conv_2d_nhwc_hwc` and
`linalg.transpose`.  Like the reference's own harness, which reads MLIR text
with regular expressions (tools/harness/verify_accuracy.py:298-359,
tools/harness/e2e_verify.py:78-140), this is a reader for that pretty-printed
subset, not a general MLIR parser: anything else is kept as an opaque op so
that uses and users stay correct.
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field

TYPE_BITS = {"f16": 16, "bf16": 16, "f32": 32, "f64": 64, "i8": 8, "i16": 16, "i32": 32,
             "i64": 64, "index": 64, "i1": 1}

_STMT_START = re.compile(
    r"^(%|return\b|func\.return\b|func\.call\b|linalg\.|tensor\.|arith\.|scf\.|memref\.|npu\.)")


@dataclass
class TType:
    shape: list          # [] for scalars, -1 for dynamic dims
    elem: str
    shaped: bool = True

    @property
    def bits(self):
        return TYPE_BITS.get(self.elem, 32)

    def __str__(self):
        if not self.shaped:
            return self.elem
        dims = "x".join("?" if d < 0 else str(d) for d in self.shape)
        return f"tensor<{dims}x{self.elem}>" if dims else f"tensor<{self.elem}>"


@dataclass
class MOp:
    name: str                          # e.g. "linalg.matmul"
    results: list                      # SSA names
    result_types: list
    ins: list = field(default_factory=list)       # SSA names
    outs: list = field(default_factory=list)
    operands: list = field(default_factory=list)  # other operand names (pad source, return values)
    iterators: list = field(default_factory=list)  # generic: "parallel" / "reduction"
    body_ops: list = field(default_factory=list)   # generic region: arith op names
    attrs: dict = field(default_factory=dict)
    text: str = ""

    @property
    def all_operands(self):
        return self.ins + self.outs + self.operands


@dataclass
class MFunc:
    name: str
    args: list          # [(name, TType)]
    result_types: list
    ops: list           # [MOp]
    types: dict         # SSA name -> TType
    target: dict = None  # the enclosing module's #npu.target parameters, if it has one


TARGET_PARAMS = ("num_cores", "sram_per_core", "dram_bandwidth", "sram_bandwidth",
                 "matrix_throughput", "dsp_throughput", "dma_channels")


def parse_target(text: str):
    """The module's `npu.target` attribute (include/npu/Dialect/NPU/NPUDialect.td:100-113:
    `#npu.target<num_cores = .., sram_per_core = .., ...>`, the seven int64
    parameters in any order), given inline in `module attributes {...}` or
    through an attribute alias (`#t = #npu.target<...>` ... `npu.target = #t`).
    Returns {param: value} or None when the module sets none."""
    m = re.search(r"\bnpu\.target\s*=\s*(#[\w.]+(?:<[^>]*>)?)", text)
    if not m:
        return None
    ref = m.group(1)
    if not ref.startswith("#npu.target<"):
        alias = re.search(r"^\s*" + re.escape(ref) + r"\s*=\s*(#npu\.target<[^>]*>)", text, re.M)
        if not alias:
            raise ValueError(f"npu.target refers to {ref}, which the text does not define")
        ref = alias.group(1)
    body = ref[len("#npu.target<"):-1]
    vals = {}
    for part in _split_top(body):
        if not part:
            continue
        k, v = (x.strip() for x in part.split("=", 1))
        if k not in TARGET_PARAMS:
            raise ValueError(f"#npu.target: unknown parameter {k}")
        vals[k] = int(v.split(":")[0].strip())
    missing = [k for k in TARGET_PARAMS if k not in vals]
    if missing:
        raise ValueError(f"#npu.target: missing {missing}")
    return vals


def parse_type(s: str) -> TType:
    s = s.strip()
    m = re.match(r"(tensor|memref)<([^>]*)>", s)
    if not m:
        return TType([], s, shaped=False)
    parts = m.group(2).split(",")[0].strip().split("x")
    elem = parts[-1]
    shape = [-1 if p == "?" else int(p) for p in parts[:-1]]
    return TType(shape, elem)


def _split_top(s: str, sep=","):
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "([{<":
            depth += 1
        elif ch in ")]}>":
            depth -= 1
        if ch == sep and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    return [x.strip() for x in out]


def _find_group(s: str, key: str):
    """Text inside the parentheses of the first top-level `key(`."""
    depth = 0
    i = 0
    while i < len(s):
        ch = s[i]
        if depth == 0 and s.startswith(key + "(", i) and (i == 0 or not s[i - 1].isalnum()):
            j = i + len(key) + 1
            d = 1
            k = j
            while k < len(s) and d:
                if s[k] == "(":
                    d += 1
                elif s[k] == ")":
                    d -= 1
                k += 1
            return s[j:k - 1]
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        i += 1
    return None


def _operand_list(group: str):
    """`%a, %b : t1, t2` -> ([names], [types])."""
    if group is None:
        return [], []
    if ":" in group:
        names, types = group.split(":", 1)
        return ([n.strip() for n in names.split(",") if n.strip()],
                [parse_type(t) for t in _split_top(types)])
    return [n.strip() for n in group.split(",") if n.strip()], []


def _strip_regions(s: str):
    """The statement with every {...} region / attribute dict removed."""
    out, depth = "", 0
    for ch in s:
        if ch == "{":
            depth += 1
            continue
        if ch == "}":
            depth -= 1
            continue
        if depth == 0:
            out += ch
    return out


def _statements(body: str):
    stmts, cur, depth = [], [], 0
    for raw in body.split("\n"):
        line = raw.split("//", 1)[0].rstrip()
        if not line.strip():
            continue
        if depth == 0 and _STMT_START.match(line.strip()) and cur:
            stmts.append("\n".join(cur))
            cur = []
        cur.append(line)
        depth += sum(line.count(c) for c in "([{") - sum(line.count(c) for c in ")]}")
    if cur:
        stmts.append("\n".join(cur))
    return stmts


@dataclass
class BodyOp:
    """One operation of a linalg.generic region: ``result = name operands``
    (``value`` holds an arith.constant's literal, ``type`` the text after the
    colon, e.g. "i64" or "i64 to i32")."""
    result: str
    name: str
    operands: list
    value: str = None
    type: str = ""


def parse_maps(attr_text: str) -> list:
    """indexing_maps -> one list of result expressions per operand, in the
    map's own dimension names replaced by their positions ("d1" -> 1; any
    other expression is kept as text)."""
    out = []
    for dims, res in re.findall(r"affine_map<\(([^)]*)\)\s*->\s*\(([^)]*)\)>", attr_text):
        names = [d.strip() for d in dims.split(",") if d.strip()]
        exprs = []
        for e in (x.strip() for x in res.split(",") if x.strip()):
            exprs.append(names.index(e) if e in names else e)
        out.append(exprs)
    return out


def parse_region(region: str):
    """A generic's region -> (block argument names, [BodyOp], yielded values)."""
    if not region:
        return [], [], []
    m = re.match(r"\^bb\d*\(([^)]*)\)\s*:", region)
    args = [a.split(":")[0].strip() for a in m.group(1).split(",")] if m else []
    body, yielded = [], []
    for line in region[m.end() if m else 0:].split("\n"):
        line = line.split("//", 1)[0].strip().rstrip("}").strip()
        if not line:
            continue
        y = re.match(r"linalg\.yield\s+(.*?)\s*:", line)
        if y:
            yielded = [v.strip() for v in y.group(1).split(",")]
            continue
        b = re.match(r"(%[\w]+)\s*=\s*([\w\.]+)\s*(.*)$", line)
        if not b:
            continue
        res, name, tail = b.groups()
        ty = tail.split(":", 1)[1].strip() if ":" in tail else ""
        if name == "arith.constant":
            body.append(BodyOp(res, name, [], tail.rsplit(":", 1)[0].strip(), ty))
        elif name == "linalg.index":  # the value is the iteration dimension
            body.append(BodyOp(res, name, [], tail.split(":", 1)[0].strip(), ty))
        elif name in ("arith.cmpi", "arith.cmpf"):  # the value is the predicate
            pred, _, ops = tail.split(":", 1)[0].partition(",")
            body.append(BodyOp(res, name, re.findall(r"%[\w]+", ops), pred.strip(), ty))
        else:
            body.append(BodyOp(res, name, re.findall(r"%[\w]+", tail.split(":", 1)[0]), None, ty))
    return args, body, yielded


def parse_op(stmt: str) -> MOp:
    s = stmt.strip()
    results = []
    m = re.match(r"^((?:%[\w]+(?::\d+)?\s*,\s*)*%[\w]+(?::\d+)?)\s*=\s*", s)
    if m:
        results = [r.strip() for r in m.group(1).split(",")]
        s = s[m.end():]
    name = re.match(r"[\w\.]+", s).group(0)
    rest = s[len(name):]
    op = MOp(name=name, results=results, result_types=[], text=stmt)
    flat = _strip_regions(rest)
    if name == "arith.constant":
        ty = flat.rsplit(":", 1)[1].strip()
        op.result_types = [parse_type(ty)]
        op.attrs["value"] = flat.rsplit(":", 1)[0].strip()
    elif name == "tensor.empty":
        op.result_types = [parse_type(flat.rsplit(":", 1)[1])]
    elif name == "tensor.pad":
        src = re.match(r"\s*(%[\w]+)", flat).group(1)
        op.operands = [src]
        lo = re.search(r"low\[([^\]]*)\]", flat)
        hi = re.search(r"high\[([^\]]*)\]", flat)
        op.attrs["low"] = [int(x) for x in lo.group(1).split(",")] if lo else []
        op.attrs["high"] = [int(x) for x in hi.group(1).split(",")] if hi else []
        m2 = re.search(r":\s*(tensor<[^>]*>)\s*to\s*(tensor<[^>]*>)", flat)
        op.result_types = [parse_type(m2.group(2))]
        op.attrs["source_type"] = parse_type(m2.group(1))
        y = re.search(r"tensor\.yield\s+(%[\w]+)", rest)
        op.attrs["yield"] = y.group(1) if y else None
    elif name in ("return", "func.return"):
        op.name = "func.return"
        names = flat.split(":", 1)[0]
        op.operands = [n.strip() for n in names.split(",") if n.strip().startswith("%")]
    elif name in ("tensor.collapse_shape", "tensor.expand_shape"):
        op.operands = [re.match(r"\s*(%[\w]+)", flat).group(1)]
        op.result_types = [parse_type(flat.rsplit("into", 1)[1])]
        ra = re.search(r"\[\s*(\[[\d,\s\[\]]*\])\s*\]", flat)
        op.attrs["reassociation"] = [[int(d) for d in grp.split(",") if d.strip()]
                                     for grp in re.findall(r"\[([\d,\s]*)\]", ra.group(1))] \
            if ra else []
        op.attrs["source_type"] = parse_type(flat.rsplit("into", 1)[0].rsplit(":", 1)[1])
    elif name == "func.call":
        m2 = re.match(r"\s*@([\w]+)\(([^)]*)\)\s*:\s*\(([^)]*)\)\s*->\s*(.*)$", flat.strip(), re.S)
        op.attrs["callee"] = m2.group(1)
        op.operands = [n.strip() for n in m2.group(2).split(",") if n.strip()]
        rt = m2.group(4).strip()
        if rt.startswith("("):
            rt = rt[1:-1]
        op.result_types = [parse_type(t) for t in _split_top(rt)] if rt else []
    elif name.startswith("linalg."):
        op.ins, in_types = _operand_list(_find_group(flat, "ins"))
        op.outs, out_types = _operand_list(_find_group(flat, "outs"))
        op.attrs["in_types"] = in_types
        op.attrs["out_types"] = out_types
        m2 = re.search(r"->\s*(.*)$", flat.strip(), re.S)
        if m2:
            rt = m2.group(1).strip()
            if rt.startswith("("):
                rt = rt[1:-1]
            op.result_types = [parse_type(t) for t in _split_top(rt)]
        elif results:
            op.result_types = list(out_types)
        if name == "linalg.generic":
            it = re.search(r"iterator_types\s*=\s*\[([^\]]*)\]", rest)
            op.iterators = re.findall(r'"(\w+)"', it.group(1)) if it else []
            region = rest[rest.rfind("^bb"):] if "^bb" in rest else ""
            op.body_ops = re.findall(r"\b(arith\.\w+|math\.\w+)", region)
            op.attrs["maps"] = parse_maps(rest[:rest.find("^bb")] if "^bb" in rest else rest)
            op.attrs["block_args"], op.attrs["body"], op.attrs["yield"] = parse_region(region)
        if name == "linalg.transpose":
            p = re.search(r"permutation\s*=\s*\[([^\]]*)\]", rest)
            op.attrs["permutation"] = [int(x) for x in p.group(1).split(",")] if p else []
        st = re.search(r"strides\s*=\s*dense<(\[[^\]]*\]|\d+)>", rest)
        if st:
            v = st.group(1)
            op.attrs["strides"] = ([int(x) for x in v.strip("[]").split(",")] if v.startswith("[")
                                   else [int(v)] * 2)
    else:
        op.operands = re.findall(r"%[\w]+", flat.split(":", 1)[0])
    return op


def split_functions(text: str) -> list:
    """Every func.func with a body: dicts of name, private (bool), header
    (the text between the argument list and the body: results and
    attributes), args [(name, TType)], result_types and body (text)."""
    funcs = []
    for m in re.finditer(r"func\.func\s+(private\s+)?@([\w]+)\s*\(", text):
        i = m.end()
        depth, j = 1, i
        while depth:
            if text[j] == "(":
                depth += 1
            elif text[j] == ")":
                depth -= 1
            j += 1
        args_txt = text[i:j - 1]
        k = text.index("{", j)
        # a `{` of an attribute dict before the body: `attributes {npu.fused_kernel} {`
        while re.search(r"attributes\s*$", text[j:k]):
            d, e = 1, k + 1
            while d:
                d += {"{": 1, "}": -1}.get(text[e], 0)
                e += 1
            k = text.index("{", e)
        header = text[j:k]
        depth, e = 1, k + 1
        while depth:
            if text[e] == "{":
                depth += 1
            elif text[e] == "}":
                depth -= 1
            e += 1
        args, arg_text = [], []
        for a in _split_top(args_txt):
            if not a:
                continue
            n, t = a.split(":", 1)
            args.append((n.strip(), parse_type(t.split("{")[0])))
            arg_text.append(t.strip())
        rtypes = []
        rm = re.search(r"->\s*(.*?)(?:attributes|$)", header, re.S)
        if rm and rm.group(1).strip():
            rt = rm.group(1).strip()
            if rt.startswith("("):
                rt = rt[1:-1]
            rtypes = [parse_type(t) for t in _split_top(rt)]
        funcs.append({"name": m.group(2), "private": bool(m.group(1)), "header": header,
                      "args": args, "arg_text": arg_text, "result_types": rtypes,
                      "body": text[k + 1:e - 1]})
    return funcs


def parse_functions(text: str) -> list:
    """Every func.func with a body in the text."""
    funcs = []
    for f in split_functions(text):
        ops = [parse_op(s) for s in _statements(f["body"])]
        types = {n: t for n, t in f["args"]}
        for op in ops:
            for r, t in zip(op.results, op.result_types):
                types[r] = t
        funcs.append(MFunc(f["name"], f["args"], f["result_types"], ops, types))
    target = parse_target(text)
    for f in funcs:
        f.target = target
    return funcs


def parse_file(path: str) -> list:
    with open(path) as f:
        return parse_functions(f.read())
