"""Lowering of a Llama decoder layer written in linalg to the four Llama entry
points (include/npu_amd.h: fused_llama_qkv_rope, fused_llama_attention,
fused_llama_matmul_residual, fused_llama_rmsnorm_swiglu).

The reference's Llama text (test/llama_attention.mlir) is an attention block
with ReLU in place of softmax and neither norm, RoPE nor gating; its passes
group such a function by the producer/consumer chains they see
(lib/Transforms/FusionPass.cpp) and its tests check the groups, not an
execution.  Here the real layer is executed: the matcher follows the values of
the function from its arguments and recognises, by what every region
computes,

* RMSNorm: a reduction generic sum(extf(x)^2) into a fill of 0.0, then a
  parallel generic truncf(extf(x) * (1 / sqrt(ss / D + eps)) * g) -- in that
  association, the oracle's `orc_rmsnorm_f32`;
* Q, K, V: three matmuls of the normalised rows into fills of 0.0; Q and K
  expanded to [S, H, Dh/2, 2], rotated by a generic that selects
  x0 c - x1 s for pair element 0 and x0 s + x1 c for element 1, truncated and
  collapsed back; V truncated -> fused_llama_qkv_rope;
* attention: per-head views (expand + transpose [1, 0, 2], K's [1, 2, 0]),
  batch_matmul Q K^T, one generic scaling by a constant and writing -inf where
  the key index exceeds the query index, the softmax as max / exp(s - max) /
  sum / divide generics, batch_matmul with V, transpose back, collapse,
  truncf -> fused_llama_attention;
* truncf(extf(r) + a @ w) -> fused_llama_matmul_residual;
* RMSNorm followed by two matmuls gate / up and truncf(g / (1 + exp(-g)) * u)
  -> fused_llama_rmsnorm_swiglu.

Anything else in such a function raises NotImplementedError naming the value
that does not fit; there is no fallback implementation.
"""
from __future__ import annotations

from . import lower as L


def _fail(v, why):
    raise NotImplementedError(f"{v}: {why}")


def _ident(n):
    return list(range(n))


def _users(fn, v):
    return [o for o in fn.f.ops if v in o.ins or v in o.operands]


def _one_user(fn, v, kind):
    us = _users(fn, v)
    if len(us) != 1 or us[0].name != kind:
        _fail(v, f"expected one user, a {kind} (users: {[u.name for u in us]})")
    return us[0]


def _generic(fn, v, n_ins, maps, iters, tmpl):
    """The generic producing v, checked: n_ins inputs, indexing maps `maps`
    (inputs then output), iterator types `iters`, yielded value matching the
    expression template `tmpl` whose placeholders $0, $1, ... name the block
    arguments of the inputs.  Returns (op, {placeholder: bound subtree})."""
    g = fn.op(v)
    if g is None or g.name != "linalg.generic":
        _fail(v, f"expected a linalg.generic, found {g.name if g else 'an argument'}")
    if len(g.ins) != n_ins or len(g.outs) != 1 or len(g.results) != 1:
        _fail(v, f"generic with {len(g.ins)} inputs, {len(g.outs)} outputs (expected {n_ins}, 1)")
    if g.attrs.get("maps") != maps:
        _fail(v, f"indexing maps {g.attrs.get('maps')} (expected {maps})")
    if g.iterators != iters:
        _fail(v, f"iterators {g.iterators} (expected {iters})")
    b = {}
    if not L._matches(L._tree(g), tmpl, b):
        _fail(v, "generic body is not the layer's formula at this point")
    for k in list(b):
        if k[1:].isdigit() and b[k] != ("arg", int(k[1:])):
            _fail(v, f"generic body reads {b[k]} where input {k[1:]} is expected")
    return g, b


def _const_of(b, key, v, what):
    t = b.get(key)
    if t is None or t[0] != "const" or t[2] != "f32":
        _fail(v, f"{what} must be an f32 constant")
    return L._float(t[1])


def _zero_fill(fn, v, what):
    f = fn.op(v)
    if f is None or f.name != "linalg.fill":
        _fail(v, f"{what} must be a linalg.fill")
    if L._const(fn, f.ins[0]) != 0.0:
        _fail(v, f"{what} must be a fill of 0.0")
    return f


def _fill_of(fn, v, value, what):
    f = fn.op(v)
    if f is None or f.name != "linalg.fill" or L._const(fn, f.ins[0]) != value:
        _fail(v, f"{what} must be a linalg.fill of {value}")
    return f


def _matmul(fn, v, kind="linalg.matmul"):
    """(op, lhs, rhs) of the matmul producing v into a fill of 0.0."""
    m = fn.op(v)
    if m is None or m.name != kind:
        _fail(v, f"expected a {kind}")
    if kind == "linalg.matmul":
        L._check_matmul(m)
    _zero_fill(fn, m.outs[0], f"{v}'s accumulator")
    if fn.ty(v).elem != "f32":
        _fail(v, "matmul must accumulate in f32")
    return m, m.ins[0], m.ins[1]


def _reshape(fn, v, kind, reassoc):
    r = fn.op(v)
    if r is None or r.name != kind:
        _fail(v, f"expected a {kind}")
    if r.attrs.get("reassociation") != reassoc:
        _fail(v, f"{kind} reassociation {r.attrs.get('reassociation')} (expected {reassoc})")
    return r, r.operands[0]


def _transpose(fn, v, perm):
    t = fn.op(v)
    if t is None or t.name != "linalg.transpose":
        _fail(v, "expected a linalg.transpose")
    if t.attrs.get("permutation") != perm:
        _fail(v, f"permutation {t.attrs.get('permutation')} (expected {perm})")
    return t, t.ins[0]


def _ext(x):
    return ("arith.extf", "bf16 to f32", x)


def _f(op, *xs):
    return (op, "f32") + tuple(xs)


def _rmsnorm(fn, v):
    """(x, g, eps, ops) when v = the bf16 RMSNorm of x scaled by g."""
    shp = fn.ty(v).shape
    if len(shp) != 2 or fn.ty(v).elem != "bf16":
        _fail(v, "RMSNorm output must be a 2-d bf16 tensor")
    D = shp[1]
    tmpl = ("arith.truncf", "f32 to bf16",
            _f("arith.mulf",
               _f("arith.mulf", _ext(("$0",)),
                  _f("arith.divf", ("const", "1.0", "f32"),
                     _f("math.sqrt", _f("arith.addf", _f("arith.divf", ("$1",), ("$D",)),
                                        ("$eps",))))),
               ("$2",)))
    g2, b = _generic(fn, v, 3, [[0, 1], [0], [1], [0, 1]], ["parallel", "parallel"], tmpl)
    if _const_of(b, "$D", v, "the mean's divisor") != float(D):
        _fail(v, f"the mean of squares must divide by the row length {D}")
    eps = _const_of(b, "$eps", v, "epsilon")
    x, ss, g = g2.ins
    if fn.ty(x).elem != "bf16" or fn.ty(g).elem != "f32" or fn.ty(g).shape != [D]:
        _fail(v, "RMSNorm takes bf16 rows and an f32 gain of the row length")
    sq = _f("arith.addf", ("$1",), _f("arith.mulf", _ext(("$0",)), _ext(("$0",))))
    g1, _ = _generic(fn, ss, 1, [[0, 1], [0]], ["parallel", "reduction"], sq)
    if g1.ins[0] != x:
        _fail(ss, f"sum of squares of {g1.ins[0]}, normalising {x}")
    fill = _zero_fill(fn, g1.outs[0], f"{ss}'s accumulator")
    return x, g, eps, [fill, g1, g2]


def _rope(fn, v, acc, cos=None, sin=None):
    """(cos, sin, ops) when v (bf16 [S, D]) is RoPE of accumulator acc over
    interleaved pairs."""
    S, D = fn.ty(acc).shape
    col, r = _reshape(fn, v, "tensor.collapse_shape", [[0], [1, 2, 3]])
    shp = fn.ty(r).shape
    if len(shp) != 4 or shp[0] != S or shp[3] != 2 or shp[1] * shp[2] * 2 != D:
        _fail(v, f"RoPE view {shp} of [{S}, {D}]")
    idx0 = ("arith.cmpi", "index", ("pred", "eq"), ("linalg.index", "index", ("dim", 3)),
            ("const", "0", "index"))
    even = _f("arith.subf", _f("arith.mulf", ("$0",), ("$2",)), _f("arith.mulf", ("$1",), ("$3",)))
    odd = _f("arith.addf", _f("arith.mulf", ("$0",), ("$3",)), _f("arith.mulf", ("$1",), ("$2",)))
    tmpl = ("arith.truncf", "f32 to bf16", ("arith.select", "f32", idx0, even, odd))
    g, _ = _generic(fn, r, 4, [[0, 1, 2, "0"], [0, 1, 2, "1"], [0, 2], [0, 2], [0, 1, 2, 3]],
                    ["parallel"] * 4, tmpl)
    x4 = g.ins[0]
    if g.ins[1] != x4:
        _fail(r, "both pair elements must come from one view")
    ex, src = _reshape(fn, x4, "tensor.expand_shape", [[0], [1, 2, 3]])
    if src != acc:
        _fail(x4, f"RoPE of {src}, expected {acc}")
    c, s = g.ins[2], g.ins[3]
    for t in (c, s):
        if fn.ty(t).elem != "f32" or fn.ty(t).shape != [S, shp[2]]:
            _fail(t, f"cos / sin tables must be f32 [{S}, {shp[2]}]")
    if cos is not None and (c, s) != (cos, sin):
        _fail(v, "Q and K must be rotated by the same tables")
    return c, s, [ex, g, col]


def _trunc(fn, v, rank):
    tmpl = ("arith.truncf", "f32 to bf16", ("$0",))
    g, _ = _generic(fn, v, 1, [_ident(rank), _ident(rank)], ["parallel"] * rank, tmpl)
    return g.ins[0], g


def _qkv(fn, xn):
    """The fused_llama_qkv_rope call whose normalised rows are xn, or None
    when xn does not feed three projections."""
    x, g1, eps, norm = _rmsnorm(fn, xn)
    mms = [u for u in _users(fn, xn)]
    if len(mms) != 3 or any(u.name != "linalg.matmul" or u.ins[0] != xn for u in mms):
        return None
    outs, ws, ops, tables = {}, {}, list(norm), None
    for m in mms:
        _matmul(fn, m.results[0])
        acc = m.results[0]
        us = _users(fn, acc)
        if len(us) != 1:
            _fail(acc, "projection with more than one user")
        ops += [fn.op(m.outs[0]), m]
        if us[0].name == "tensor.expand_shape":
            col = _one_user(fn, _one_user(fn, us[0].results[0], "linalg.generic").results[0],
                            "tensor.collapse_shape")
            c, s, rops = _rope(fn, col.results[0], acc, *(tables or (None, None)))
            tables = (c, s)
            role = "Q" if "Q" not in outs else "K"
            outs[role], ws[role] = col.results[0], m.ins[1]
            ops += rops
        else:
            v = us[0].results[0]
            src, tg = _trunc(fn, v, 2)
            if "V" in outs:
                _fail(v, "two unrotated projections")
            outs["V"], ws["V"] = v, m.ins[1]
            ops.append(tg)
    if set(outs) != {"Q", "K", "V"}:
        _fail(xn, f"projections {sorted(outs)} (expected rotated Q, K and plain V)")
    # Q is the rotated projection that attention reads as the query
    q, k = outs["Q"], outs["K"]
    return {"entry": "fused_llama_qkv_rope", "ops": ops,
            "args": [x, g1, None, None, ws["V"], tables[0], tables[1]],
            "rot": [(q, ws["Q"]), (k, ws["K"])], "outs": [q, k, outs["V"]],
            "params": {"eps": eps}}


def _heads(fn, v, perm):
    """The [S, D] bf16 tensor of which v is the per-head view by `perm`."""
    t, e = _transpose(fn, v, perm)
    ex, src = _reshape(fn, e, "tensor.expand_shape", [[0], [1, 2]])
    S, H, Dh = fn.ty(e).shape
    if fn.ty(src).shape != [S, H * Dh] or fn.ty(src).elem != "bf16":
        _fail(e, "per-head view of a bf16 [S, D] tensor expected")
    return src, [ex, t]


def _attention(fn, a):
    """The fused_llama_attention call producing A = a (bf16 [S, D])."""
    o2, tg = _trunc(fn, a, 2)
    col, ot = _reshape(fn, o2, "tensor.collapse_shape", [[0], [1, 2]])
    tr, o = _transpose(fn, ot, [1, 0, 2])
    pv, p, vh = _matmul(fn, o, "linalg.batch_matmul")
    H, S, Dh = fn.ty(o).shape
    id3, row = [0, 1, 2], [0, 1]
    gp, _ = _generic(fn, p, 2, [id3, row, id3], ["parallel"] * 3, _f("arith.divf", ("$0",), ("$1",)))
    ex_v, l = gp.ins
    gl, _ = _generic(fn, l, 1, [id3, row], ["parallel", "parallel", "reduction"],
                     _f("arith.addf", ("$1",), ("$0",)))
    if gl.ins[0] != ex_v:
        _fail(l, "softmax sum over another tensor")
    _zero_fill(fn, gl.outs[0], f"{l}'s accumulator")
    gx, _ = _generic(fn, ex_v, 2, [id3, row, id3], ["parallel"] * 3,
                     _f("math.exp", _f("arith.subf", ("$0",), ("$1",))))
    sm, m = gx.ins
    gm, _ = _generic(fn, m, 1, [id3, row], ["parallel", "parallel", "reduction"],
                     _f("arith.maximumf", ("$1",), ("$0",)))
    if gm.ins[0] != sm:
        _fail(m, "softmax max over another tensor")
    _fill_of(fn, gm.outs[0], float("-inf"), f"{m}'s accumulator")
    masked = None
    for cmp in (("ugt", 2, 1), ("sgt", 2, 1), ("ult", 1, 2), ("slt", 1, 2)):
        pred = ("arith.cmpi", "index", ("pred", cmp[0]), ("linalg.index", "index", ("dim", cmp[1])),
                ("linalg.index", "index", ("dim", cmp[2])))
        tmpl = ("arith.select", "f32", pred, ("$ninf",), _f("arith.mulf", ("$0",), ("$scale",)))
        try:
            masked = _generic(fn, sm, 1, [id3, id3], ["parallel"] * 3, tmpl)
            break
        except NotImplementedError:
            continue
    if masked is None:
        _fail(sm, "expected scale, then -inf where the key index exceeds the query index")
    gs, b = masked
    if _const_of(b, "$ninf", sm, "the mask value") != float("-inf"):
        _fail(sm, "masked scores must be -inf")
    scale = _const_of(b, "$scale", sm, "the score scale")
    s = gs.ins[0]
    qk, qh, kt = _matmul(fn, s, "linalg.batch_matmul")
    Q, qops = _heads(fn, qh, [1, 0, 2])
    K, kops = _heads(fn, kt, [1, 2, 0])
    V, vops = _heads(fn, vh, [1, 0, 2])
    if Dh not in (64, 128) or fn.ty(s).shape != [H, S, S]:
        _fail(s, f"attention over heads of {Dh} (the entry point's head dimensions are 64 and 128)")
    ops = qops + kops + vops + [fn.op(qk.outs[0]), qk, gs, fn.op(gm.outs[0]), gm, gx,
                                fn.op(gl.outs[0]), gl, gp, fn.op(pv.outs[0]), pv, tr, col, tg]
    return {"entry": "fused_llama_attention", "ops": ops, "args": [Q, K, V], "outs": [a],
            "params": {"n_heads": H, "scale": scale}}


def _residual(fn, v):
    """(r, acc) when v = truncf(extf(r) + acc), both [S, N]."""
    tmpl = ("arith.truncf", "f32 to bf16", _f("arith.addf", _ext(("$0",)), ("$1",)))
    g, _ = _generic(fn, v, 2, [[0, 1]] * 3, ["parallel", "parallel"], tmpl)
    return g.ins[0], g.ins[1], g


def _matmul_residual(fn, v):
    r, acc, g = _residual(fn, v)
    m, a, w = _matmul(fn, acc)
    if fn.ty(a).elem != "bf16" or fn.ty(w).elem != "bf16" or fn.ty(r).elem != "bf16":
        _fail(v, "residual projection takes bf16 rows, weights and residual")
    return {"entry": "fused_llama_matmul_residual", "ops": [fn.op(m.outs[0]), m, g],
            "args": [a, w, r], "outs": [v], "params": {}}


def _swiglu(fn, v):
    """The fused_llama_rmsnorm_swiglu call producing act = v."""
    silu = _f("arith.divf", ("$0",), _f("arith.addf", ("const", "1.0", "f32"),
                                        _f("math.exp", _f("arith.negf", ("$0",)))))
    tmpl = ("arith.truncf", "f32 to bf16", _f("arith.mulf", silu, ("$1",)))
    g, _ = _generic(fn, v, 2, [[0, 1]] * 3, ["parallel", "parallel"], tmpl)
    mg, hn, wg = _matmul(fn, g.ins[0])
    mu, hn2, wu = _matmul(fn, g.ins[1])
    if hn2 != hn:
        _fail(v, "gate and up projections of different rows")
    h, g2, eps, norm = _rmsnorm(fn, hn)
    if len(_users(fn, hn)) != 2:
        _fail(hn, "normalised rows with users other than the gate and up projections")
    return {"entry": "fused_llama_rmsnorm_swiglu",
            "ops": norm + [fn.op(mg.outs[0]), mg, fn.op(mu.outs[0]), mu, g],
            "args": [h, g2, wg, wu], "outs": [v], "params": {"eps": eps}}


def _is_rmsnorm(fn, op):
    try:
        _rmsnorm(fn, op.results[0])
        return True
    except NotImplementedError:
        return False


def llama_calls(fn) -> list:
    """The Llama entry-point calls of function fn (a lower._Fn), in dataflow
    order, as dicts {entry, ops, args, outs, params}; [] when fn holds no
    batch_matmul.  Raises NotImplementedError when a batch_matmul is not on
    an attention chain the matcher recognises."""
    ops = fn.f.ops
    if not any(o.name == "linalg.batch_matmul" for o in ops):
        return []
    calls = []
    for op in ops:
        if op.name != "linalg.generic" or not op.results:
            continue
        v = op.results[0]
        if _is_rmsnorm(fn, op):
            c = _qkv(fn, v)
            if c is not None:
                # Q is the rotated tensor attention reads through the query view
                attn_q = [u for u in ops if u.name == "tensor.expand_shape"]
                (q, wq), (k, wk) = c["rot"]
                for e in attn_q:
                    if e.operands[0] == k:
                        t = _one_user(fn, e.results[0], "linalg.transpose")
                        if t.attrs.get("permutation") == [1, 0, 2]:
                            (q, wq), (k, wk) = (k, wk), (q, wq)
                c["args"][2:4] = [wq, wk]
                c["outs"] = [q, k, c["outs"][2]]
                del c["rot"]
                calls.append(c)
            continue
        body = L._tree(op)
        if body[0] == "arith.truncf" and len(op.ins) == 1:
            src = fn.op(op.ins[0])
            if src is not None and src.name == "tensor.collapse_shape":
                inner = fn.op(src.operands[0])
                if inner is not None and inner.name == "linalg.transpose":
                    calls.append(_attention(fn, v))
                    continue
        if body[0] == "arith.truncf" and len(op.ins) == 2:
            b = body[2]
            if b[0] == "arith.addf":
                calls.append(_matmul_residual(fn, v))
            elif b[0] == "arith.mulf":
                calls.append(_swiglu(fn, v))
    return calls
