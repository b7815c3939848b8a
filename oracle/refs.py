"""Oracle results and error-bound magnitudes for each workload's inputs.

TEST INFRASTRUCTURE ONLY (see oracle.py).  ``reference(name, inputs)`` runs
the unfused CPU restatement of the workload's linalg chain and returns
``{output_name: (expected, mag)}`` where ``mag`` is the chain evaluated on
absolute values (the scale of the per-element error bound) or None for
integer outputs that must match bit for bit.  ``run_oracle`` runs only the
restatement (what the CPU baseline times).
"""
from __future__ import annotations

import numpy as np

import oracle


def _bf(x):
    return (np.ascontiguousarray(x, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _absf(x):
    if x.dtype == np.uint16:
        return np.abs(_bf(x))
    return np.abs(np.asarray(x, np.float32))


def _sel(images):
    if images is None:
        return lambda a: a
    return lambda a: np.ascontiguousarray(a[list(images)])


# ------------------------------------------------------------ per group
def matmul_bias_act(A, B, bias, act="relu"):
    out = oracle.block_matmul_bias_act(A, B, bias, act)
    mag = np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)
    if bias is not None:
        mag = mag + np.abs(bias)
    return out, mag


def conv_bias_act(x, w, bias, pad=1, act="relu"):
    out = oracle.block_conv_bias_act(x, w, bias, pad, act)
    ax = oracle.pad_nhwc(_absf(x), (pad, pad, pad, pad))
    mag = oracle.conv2d_nhwc_fhwc(ax, _absf(w)).astype(np.float64)
    if bias is not None:
        mag = mag + np.abs(bias)
    return out, mag


def conv_nchw_act(x, w, bias=None, res=None, pad=1, act="relu", stride=1):
    """One NCHW conv group as the oracle runs it: tensor.pad, fill 0,
    conv_2d_nchw_fchw (strided), then bias, residual and activation
    generics; mag is the same chain on absolute values."""
    st = (stride, stride)
    xp = oracle.pad_nchw(x, (pad, pad, pad, pad)) if pad else np.asarray(x, np.float32)
    out = oracle.conv2d_nchw_fchw(xp, w, st)
    axp = oracle.pad_nchw(np.abs(x), (pad, pad, pad, pad)) if pad else np.abs(x)
    mag = oracle.conv2d_nchw_fchw(axp, np.abs(w), st).astype(np.float64)
    if bias is not None:
        out = oracle.add(out, np.broadcast_to(np.asarray(bias, np.float32)[None, :, None, None],
                                              out.shape))
        mag = mag + np.abs(bias)[None, :, None, None]
    if res is not None:
        out = oracle.add(out, res)
        mag = mag + np.abs(res)
    if act == "relu":
        out = oracle.relu(out)
    elif act == "relu6":
        out = oracle.relu6(out)
    return out, mag


def nchw_workload(name, args):
    """The oracle's result and magnitude bound for the reference's NCHW conv
    workloads (test/conv2d_relu.mlir, test/resnet_block.mlir,
    test/resnet50_block.mlir, test/mobilenet_block.mlir) on argument arrays
    in the function's order; a later conv's bound carries the earlier
    stage's through its filter (conv of the magnitude)."""
    if name == "conv2d_relu.mlir":
        x, w = args
        return conv_nchw_act(x, w, pad=1)
    if name == "resnet_block.mlir":
        x, w1, w2 = args
        r1, m1 = conv_nchw_act(x, w1, pad=1)
        out, _ = conv_nchw_act(r1, w2, res=x, pad=1, act="none")
        mag = oracle.conv2d_nchw_fchw(oracle.pad_nchw(m1, (1, 1, 1, 1)), np.abs(w2)) + np.abs(x)
        return out, mag.astype(np.float64)
    x, w1, w2, w3 = args
    r1, m1 = conv_nchw_act(x, w1, pad=0)
    r2, _ = conv_nchw_act(r1, w2, pad=1)
    m2 = oracle.conv2d_nchw_fchw(oracle.pad_nchw(m1, (1, 1, 1, 1)), np.abs(w2))
    act = "relu" if name == "resnet50_block.mlir" else "none"
    out, _ = conv_nchw_act(r2, w3, res=x, pad=0, act=act)
    mag = oracle.conv2d_nchw_fchw(m2, np.abs(w3)) + np.abs(x)
    return out, mag.astype(np.float64)


def _generic_kind(op):
    """'relu' or 'add' for the model zoo's two epilogue generics, by body."""
    body = [b.name for b in op.attrs.get("body", [])]
    if "arith.maximumf" in body and len(op.ins) == 1:
        return "relu"
    if body[:1] == ["arith.addf"] and len(op.ins) == 2:
        return "add"
    raise NotImplementedError(f"{op.results[0]}: generic body {body}")


def run_network(func, args, given=None):
    """Runs a parsed linalg function of the model zoo's forms (NCHW
    conv_2d_nchw_fchw with strides, matmul, zero fills and pads, ReLU and
    add generics) op by op with the oracle's loops, the way mlir-runner runs
    the lowered function.  ``given`` maps SSA names to values computed
    elsewhere (the GPU's results of earlier launches): an op reads a given
    value instead of the oracle's own, so each op's result is the oracle's
    for the same inputs.  Returns (vals, mags, depth) by SSA name: mags is
    the same computation on magnitudes, restarted at every given value (each
    conv / matmul applied to its inputs' magnitudes and the filters'
    absolute values, adds summed, ReLU passed through), the scale of the
    value's error bound; depth counts conv / matmul ops since the last given
    value."""
    given = given or {}
    vals, mags, depth = {}, {}, {}

    def src(v):
        if v in given:
            x = np.asarray(given[v], np.float32)
            return x, np.abs(x), 0
        return vals[v], mags[v], depth[v]
    for (a, _), x in zip(func.args, args):
        vals[a] = np.asarray(x, np.float32)
        mags[a] = np.abs(vals[a])
        depth[a] = 0
    for op in func.ops:
        r = op.results[0] if op.results else None
        if op.name in ("arith.constant", "tensor.empty", "linalg.fill", "func.return"):
            continue
        if op.name == "tensor.pad":
            lo, hi = op.attrs["low"], op.attrs["high"]
            x, m, d = src(op.operands[0])
            pads = (lo[2], hi[2], lo[3], hi[3])
            vals[r], mags[r], depth[r] = oracle.pad_nchw(x, pads), oracle.pad_nchw(m, pads), d
        elif op.name == "linalg.conv_2d_nchw_fchw":
            (x, mx, dx), (w, mw, dw) = src(op.ins[0]), src(op.ins[1])
            st = tuple(op.attrs.get("strides", [1, 1]))
            vals[r] = oracle.conv2d_nchw_fchw(x, w, st)
            mags[r] = oracle.conv2d_nchw_fchw(mx, mw, st)
            depth[r] = max(dx, dw) + 1
        elif op.name == "linalg.matmul":
            (a, ma, da), (b, mb, db) = src(op.ins[0]), src(op.ins[1])
            vals[r], mags[r], depth[r] = oracle.matmul(a, b), oracle.matmul(ma, mb), max(da, db) + 1
        elif op.name == "linalg.generic":
            if _generic_kind(op) == "relu":
                x, m, d = src(op.ins[0])
                vals[r], mags[r], depth[r] = oracle.relu(x), m, d
            else:
                (a, ma, da), (b, mb, db) = src(op.ins[0]), src(op.ins[1])
                vals[r], mags[r], depth[r] = oracle.add(a, b), ma + mb, max(da, db)
        else:
            raise NotImplementedError(op.name)
    return vals, {k: v.astype(np.float64) for k, v in mags.items()}, depth


def irb(x, we, wdw, wp):
    out = oracle.block_irb(x, we, wdw, wp)
    ax = np.abs(x)
    me = oracle.conv2d_nhwc_fhwc(ax, np.abs(we)[:, None, None, :])
    md = oracle.depthwise_conv2d_nhwc_hwc(oracle.pad_nhwc(me, (1, 1, 1, 1)), np.abs(wdw))
    mag = oracle.conv2d_nhwc_fhwc(md, np.abs(wp)[:, None, None, :]).astype(np.float64) + ax
    return out, mag


def qbottleneck(inp, images=None):
    s = _sel(images)
    return oracle.block_qbottleneck(s(inp["x"]), inp["w1"], inp["w2"], inp["w3"], inp["m1"],
                                    inp["s1"], inp["m2"], inp["s2"], inp["m3"], inp["s3"])


# ------------------------------------------------------------ Llama layer
LLAMA_HEADS, LLAMA_EPS = 8, 1e-5


def _f64(x):
    return _bf(x).astype(np.float64) if x.dtype == np.uint16 else np.asarray(x, np.float64)


def llama_stages(inp, H, eps):
    """The oracle's five sub-group outputs of one decoder layer."""
    x = inp["x"]
    S, D = x.shape
    Q, K, V = oracle.llama_qkv(x, inp["g1"], inp["wq"], inp["wk"], inp["wv"], inp["cos_t"],
                               inp["sin_t"], H, eps)
    A = oracle.llama_attention(Q, K, V, H, float((D // H) ** -0.5))
    h = oracle.llama_matmul_residual(A, inp["wo"], x)
    act = oracle.llama_swiglu(h, inp["g2"], inp["wg"], inp["wu"], eps)
    out = oracle.llama_matmul_residual(act, inp["wd"], h)
    return {"Q": Q, "K": K, "V": V, "A": A, "h": h, "act": act, "out": out}


def normed_bf16(x, g, eps):
    """bf16(rmsnorm(x) * g) exactly as the oracle's sub-groups form the matmul input."""
    return oracle.trunc_bf16(oracle.rmsnorm(oracle.ext_bf16(x), g, eps))


def mag_qkv(xn, w, cos_t, sin_t, rope):
    m = np.abs(_f64(xn)) @ np.abs(_f64(w))
    if not rope:
        return m
    S, D = m.shape
    mp = m.reshape(S, D // 2, 2)
    Dh = 2 * cos_t.shape[1]
    c = np.abs(np.tile(cos_t, (1, D // Dh))).astype(np.float64)
    s = np.abs(np.tile(sin_t, (1, D // Dh))).astype(np.float64)
    out = np.empty_like(mp)
    out[..., 0] = mp[..., 0] * c + mp[..., 1] * s
    out[..., 1] = mp[..., 0] * s + mp[..., 1] * c
    return out.reshape(S, D)


def mag_attention(Q, K, V, H):
    q, k, v = _f64(Q), _f64(K), _f64(V)
    S, D = q.shape
    Dh = D // H
    mag = np.empty((S, D))
    mask = np.triu(np.ones((S, S), bool), 1)
    for h in range(H):
        sl = slice(h * Dh, (h + 1) * Dh)
        s = (q[:, sl] @ k[:, sl].T) * Dh ** -0.5
        s[mask] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        mag[:, sl] = p @ np.abs(v[:, sl])
    return mag


def mag_residual(a, w, res):
    return np.abs(_f64(res)) + np.abs(_f64(a)) @ np.abs(_f64(w))


def mag_swiglu(hn, wg, wu):
    g, u = _f64(hn) @ _f64(wg), _f64(hn) @ _f64(wu)
    mg, mu = np.abs(_f64(hn)) @ np.abs(_f64(wg)), np.abs(_f64(hn)) @ np.abs(_f64(wu))
    sg = g / (1 + np.exp(-g))
    return mg * np.abs(u) + np.abs(sg) * mu + np.abs(sg * u)


def _rope64(m, cos_t, sin_t):
    S, D = m.shape
    Dh = 2 * cos_t.shape[1]
    c = np.tile(np.asarray(cos_t, np.float64), (1, D // Dh))
    s = np.tile(np.asarray(sin_t, np.float64), (1, D // Dh))
    mp = m.reshape(S, D // 2, 2)
    out = np.empty_like(mp)
    out[..., 0] = mp[..., 0] * c - mp[..., 1] * s
    out[..., 1] = mp[..., 0] * s + mp[..., 1] * c
    return out.reshape(S, D)


def llama_stage_exact(inp, st, H, eps):
    """Each sub-group's value in float64 before its output rounding, from the
    bf16 inputs the stage tests give the GPU (the oracle's previous stage
    outputs; the normalised rows as the oracle forms them): the reference
    point of the rounding-aware stage bound."""
    x = inp["x"]
    S, D = x.shape
    Dh = D // H
    xn = _f64(normed_bf16(x, inp["g1"], eps))
    out = {"Q": _rope64(xn @ _f64(inp["wq"]), inp["cos_t"], inp["sin_t"]),
           "K": _rope64(xn @ _f64(inp["wk"]), inp["cos_t"], inp["sin_t"]),
           "V": xn @ _f64(inp["wv"])}
    q, k, v = _f64(st["Q"]), _f64(st["K"]), _f64(st["V"])
    A = np.empty((S, D))
    mask = np.triu(np.ones((S, S), bool), 1)
    for h in range(H):
        sl = slice(h * Dh, (h + 1) * Dh)
        sc = (q[:, sl] @ k[:, sl].T) * Dh ** -0.5
        sc[mask] = -np.inf
        p = np.exp(sc - sc.max(1, keepdims=True))
        A[:, sl] = (p / p.sum(1, keepdims=True)) @ v[:, sl]
    out["A"] = A
    out["h"] = _f64(x) + _f64(st["A"]) @ _f64(inp["wo"])
    hn = _f64(normed_bf16(st["h"], inp["g2"], eps))
    g, u = hn @ _f64(inp["wg"]), hn @ _f64(inp["wu"])
    out["act"] = g / (1 + np.exp(-g)) * u
    out["out"] = _f64(st["h"]) + _f64(st["act"]) @ _f64(inp["wd"])
    return out


def llama_reference(inp, H, eps):
    """{name: (expected, mag)} for the layer's h and out."""
    st = llama_stages(inp, H, eps)
    hn = normed_bf16(st["h"], inp["g2"], eps)
    m_h = mag_residual(st["A"], inp["wo"], inp["x"])
    m_act = mag_swiglu(hn, inp["wg"], inp["wu"])
    m_out = np.abs(_f64(st["h"])) + m_h + m_act @ np.abs(_f64(inp["wd"]))
    return {"h": (st["h"], m_h), "out": (st["out"], m_out)}


# ------------------------------------------------------------ registry
def run_oracle(workload_name: str, inp: dict, images=None) -> dict:
    s = _sel(images)
    if workload_name.startswith("matmul_bias_relu"):
        return {"out": oracle.block_matmul_bias_act(inp["A"], inp["B"], inp["bias"], "relu")}
    if workload_name.startswith("conv3x3_bias_relu"):
        return {"out": oracle.block_conv_bias_act(s(inp["x"]), inp["w"], inp["bias"], 1, "relu")}
    if workload_name.startswith("mbv2_irb"):
        return {"out": oracle.block_irb(s(inp["x"]), inp["we"], inp["wdw"], inp["wp"])}
    if workload_name.startswith("qbottleneck"):
        return {"out": qbottleneck(inp, images)}
    if workload_name.startswith("llama_layer"):
        st = oracle.block_llama_layer(inp["x"], inp["g1"], inp["g2"], inp["wq"], inp["wk"],
                                      inp["wv"], inp["wo"], inp["wg"], inp["wu"], inp["wd"],
                                      inp["cos_t"], inp["sin_t"], LLAMA_HEADS, LLAMA_EPS)
        return {"h": st[0], "out": st[1]}
    raise KeyError(workload_name)


def reference(workload_name: str, inp: dict, images=None) -> dict:
    """Expected outputs of a named workload; ``images`` restricts batched
    workloads to a subset of batch indices (each image is independent)."""
    s = _sel(images)
    if workload_name.startswith("matmul_bias_relu"):
        return {"out": matmul_bias_act(inp["A"], inp["B"], inp["bias"], "relu")}
    if workload_name.startswith("conv3x3_bias_relu"):
        return {"out": conv_bias_act(s(inp["x"]), inp["w"], inp["bias"], 1, "relu")}
    if workload_name.startswith("mbv2_irb"):
        return {"out": irb(s(inp["x"]), inp["we"], inp["wdw"], inp["wp"])}
    if workload_name.startswith("qbottleneck"):
        return {"out": (qbottleneck(inp, images), None)}
    if workload_name.startswith("llama_layer"):
        return llama_reference(inp, LLAMA_HEADS, LLAMA_EPS)
    raise KeyError(workload_name)
