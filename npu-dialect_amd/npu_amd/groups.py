"""Python mirror of the fused-group entry points (include/npu_amd.h).

Each function takes torch tensors that already live on the GPU, builds the
npu_memref descriptors and calls the extern "C" entry point on the current
torch stream (or the given one).  A non-OK status raises NpuError with the
library's own message; nothing falls back to another implementation.

The group names follow the op chains the reference's outliner groups
(lib/Transforms/OutlineFusedGroupsPass.cpp:259-263): see ``OUTLINED_NAMES``.
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from .memref import absent, from_tensor, ref
from .names import OUTLINED_NAMES  # noqa: F401  (re-exported)

ACT = {"none": 0, "relu": 1, "relu6": 2}

class NpuError(RuntimeError):
    def __init__(self, status: int, where: str):
        lib = _lib.lib()
        msg = lib.npu_last_error().decode()
        name = lib.npu_status_string(status).decode()
        super().__init__(f"{where}: {name} ({status}): {msg}")
        self.status = status


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return getattr(stream, "cuda_stream", stream)


_plan_log = None


class collect_plans:
    """Context manager: gathers the launch plans of every entry-point call made
    inside it (in call order) into ``.plans``."""

    def __enter__(self):
        global _plan_log
        self.plans = []
        self._prev, _plan_log = _plan_log, self.plans
        return self

    def __exit__(self, *exc):
        global _plan_log
        _plan_log = self._prev
        return False


def _check(status, where):
    if status != 0:
        raise NpuError(status, where)
    if _plan_log is not None:
        _plan_log.extend(_lib.last_launch_plans())


def _opt(t):
    return absent() if t is None else from_tensor(t)


def fused_matmul_bias_act(A, B, bias, out, act="relu", stream=None):
    """out = act(A @ B + bias); f32 [M,K] @ [K,N] (+ [N])."""
    mA, mB, mb, mo = from_tensor(A), from_tensor(B), _opt(bias), from_tensor(out)
    st = _lib.lib().fused_matmul_bias_act(ref(mA), ref(mB), ref(mb), ref(mo), ACT[act],
                                          _stream(stream))
    _check(st, "fused_matmul_bias_act")
    return out


def _dump_ptr(lds_dump, plan):
    """The device address the launch copies a workgroup's LDS to: the kernel
    writes plan.lds_bytes bytes there, so the tensor must hold them."""
    if lds_dump is None:
        return None
    if not lds_dump.is_cuda or not lds_dump.is_contiguous() or \
            lds_dump.numel() * lds_dump.element_size() < plan.lds_bytes:
        raise ValueError(f"lds_dump: a contiguous device tensor of at least {plan.lds_bytes} "
                         "bytes is needed")
    return lds_dump.data_ptr()


def planned_matmul_bias_act(A, B, bias, out, plan, act="relu", lds_dump=None, stream=None):
    """out = act(A @ B + bias) as the reference's bufferized tile loop, every
    SRAM buffer at the LDS offset `plan` (an NpuTilePlan, see
    npu_amd.tileplan) gives it; `lds_dump` (a device tensor of
    plan.lds_bytes bytes) receives tile (0, 0)'s LDS at the end."""
    mA, mB, mb, mo = from_tensor(A), from_tensor(B), _opt(bias), from_tensor(out)
    dump = _dump_ptr(lds_dump, plan)
    st = _lib.lib().npu_planned_matmul_bias_act(ref(mA), ref(mB), ref(mb), ref(mo), ACT[act],
                                                C.byref(plan), dump, _stream(stream))
    _check(st, "npu_planned_matmul_bias_act")
    return out


def planned_conv2d_nchw_bias_act(x, w, bias, out, plan, act="relu", lds_dump=None, stream=None):
    """out = act(conv_2d_nchw_fchw(x, w) + bias) (x padded, stride 1) as the
    reference's tile loop over output-channel tiles, every SRAM buffer at
    the LDS offset `plan` (an NpuConvTilePlan, see npu_amd.tileplan) gives
    it, the next tiles' filters through its prefetch region; `lds_dump` (a
    device tensor of plan.lds_bytes bytes) receives workgroup 0's LDS at
    the end."""
    mx, mw, mb, mo = from_tensor(x), from_tensor(w), _opt(bias), from_tensor(out)
    dump = _dump_ptr(lds_dump, plan)
    st = _lib.lib().npu_planned_conv2d_nchw_bias_act(ref(mx), ref(mw), ref(mb), ref(mo), ACT[act],
                                                     C.byref(plan), dump, _stream(stream))
    _check(st, "npu_planned_conv2d_nchw_bias_act")
    return out


def fused_conv2d_nhwc_bias_act(x, w, bias, out, pad=1, act="relu", stream=None):
    """out = act(conv_2d_nhwc_fhwc(pad(x), w) + bias); f32 or bf16."""
    mx, mw, mb, mo = from_tensor(x), from_tensor(w), _opt(bias), from_tensor(out)
    st = _lib.lib().fused_conv2d_nhwc_bias_act(ref(mx), ref(mw), ref(mb), ref(mo), int(pad),
                                               ACT[act], _stream(stream))
    _check(st, "fused_conv2d_nhwc_bias_act")
    return out


def fused_conv2d_nhwc_bias_res_act(x, w, bias, res, out, pad=1, act="relu", stream=None):
    """out = act(conv_2d_nhwc_fhwc(pad(x), w) + bias + res); f32 or bf16."""
    mx, mw, mb, mr, mo = from_tensor(x), from_tensor(w), _opt(bias), from_tensor(res), from_tensor(out)
    st = _lib.lib().fused_conv2d_nhwc_bias_res_act(ref(mx), ref(mw), ref(mb), ref(mr), ref(mo),
                                                   int(pad), ACT[act], _stream(stream))
    _check(st, "fused_conv2d_nhwc_bias_res_act")
    return out


def fused_conv2d_nchw_bias_act(x, w, bias, out, pad=1, act="relu", stream=None, stride=1):
    """out = act(conv_2d_nchw_fchw(pad(x), w, stride) + bias); f32, NCHW / FCHW."""
    mx, mw, mb, mo = from_tensor(x), from_tensor(w), _opt(bias), from_tensor(out)
    st = _lib.lib().fused_conv2d_nchw_bias_act(ref(mx), ref(mw), ref(mb), ref(mo), int(pad),
                                               int(stride), ACT[act], _stream(stream))
    _check(st, "fused_conv2d_nchw_bias_act")
    return out


def fused_conv2d_nchw_bias_res_act(x, w, bias, res, out, pad=1, act="relu", stream=None,
                                   stride=1):
    """out = act(conv_2d_nchw_fchw(pad(x), w, stride) + bias + res); f32, NCHW / FCHW."""
    mx, mw, mb, mr, mo = from_tensor(x), from_tensor(w), _opt(bias), from_tensor(res), from_tensor(out)
    st = _lib.lib().fused_conv2d_nchw_bias_res_act(ref(mx), ref(mw), ref(mb), ref(mr), ref(mo),
                                                   int(pad), int(stride), ACT[act], _stream(stream))
    _check(st, "fused_conv2d_nchw_bias_res_act")
    return out


def fused_qbottleneck_i8(x, w1, w2, w3, m1, s1, m2, s2, m3, s3, out, stream=None):
    """int8 bottleneck: three convs with per-channel requant, residual, ReLU."""
    ms = [from_tensor(t) for t in (x, w1, w2, w3, m1, s1, m2, s2, m3, s3, out)]
    st = _lib.lib().fused_qbottleneck_i8(*[ref(m) for m in ms], _stream(stream))
    _check(st, "fused_qbottleneck_i8")
    return out


def fused_irb_f32(x, we, wdw, wp, out, stream=None):
    """MobileNetV2 inverted residual: expand, ReLU6, depthwise 3x3, ReLU6, project, +x."""
    ms = [from_tensor(t) for t in (x, we, wdw, wp, out)]
    st = _lib.lib().fused_irb_f32(*[ref(m) for m in ms], _stream(stream))
    _check(st, "fused_irb_f32")
    return out


def fused_llama_qkv_rope(x, g1, wq, wk, wv, cos_t, sin_t, Q, K, V, eps=1e-5, stream=None):
    """Q, K, V = rope(rmsnorm(x)*g1 @ wq), rope(... @ wk), (... @ wv); bf16."""
    ms = [from_tensor(t) for t in (x, g1, wq, wk, wv, cos_t, sin_t, Q, K, V)]
    st = _lib.lib().fused_llama_qkv_rope(*[ref(m) for m in ms], float(eps), _stream(stream))
    _check(st, "fused_llama_qkv_rope")
    return Q, K, V


def fused_llama_attention(Q, K, V, A, n_heads, scale, stream=None):
    """A = causal softmax(Q K^T * scale) V per head (head dim 64); bf16."""
    ms = [from_tensor(t) for t in (Q, K, V, A)]
    st = _lib.lib().fused_llama_attention(*[ref(m) for m in ms], int(n_heads), float(scale),
                                          _stream(stream))
    _check(st, "fused_llama_attention")
    return A


def fused_llama_matmul_residual(a, w, res, out, stream=None):
    """out = res + a @ w; bf16."""
    ms = [from_tensor(t) for t in (a, w, res, out)]
    st = _lib.lib().fused_llama_matmul_residual(*[ref(m) for m in ms], _stream(stream))
    _check(st, "fused_llama_matmul_residual")
    return out


def fused_llama_rmsnorm_swiglu(h, g2, wg, wu, act, eps=1e-5, stream=None):
    """act = silu(rmsnorm(h)*g2 @ wg) * (rmsnorm(h)*g2 @ wu); bf16."""
    ms = [from_tensor(t) for t in (h, g2, wg, wu, act)]
    st = _lib.lib().fused_llama_rmsnorm_swiglu(*[ref(m) for m in ms], float(eps), _stream(stream))
    _check(st, "fused_llama_rmsnorm_swiglu")
    return act


class Empty:
    """A tensor.empty argument of an outlined group: a shape and element type,
    and optionally the tensor that holds it (None: no data; the group never
    reads it)."""

    def __init__(self, shape, dtype="f32", tensor=None):
        self.shape, self.dtype, self.tensor = list(shape), dtype, tensor


_DT = {"f32": 0, "bf16": 1, "i8": 2, "i32": 3}


def _group_arg(x, keep):
    """One npu_arg for a tensor, an Empty or a scalar fill value."""
    a = _lib.NpuArg()
    if isinstance(x, (int, float)):
        a.kind, a.dtype, a.scalar, a.rank = 1, _DT["f32"], float(x), 0
        return a
    if isinstance(x, Empty):
        if x.tensor is not None:
            return _group_arg(x.tensor, keep)
        shape, dtype, ptr, offset, strides = x.shape, _DT[x.dtype], 0, 0, None
    else:
        m = from_tensor(x)
        shape, dtype, ptr, offset = list(x.shape), m.dtype, m.aligned, m.offset
        strides = list(x.stride())
    if strides is None:
        strides = [1] * len(shape)
        for i in range(len(shape) - 2, -1, -1):
            strides[i] = strides[i + 1] * shape[i + 1]
    d = _lib.strided_memref_type(len(shape))()
    d.allocated = d.aligned = ptr
    d.offset = offset
    for i, (sz, st) in enumerate(zip(shape, strides)):
        d.sizes[i], d.strides[i] = sz, st
    keep.append(d)
    a.rank, a.descriptor, a.dtype, a.kind = len(shape), C.addressof(d), dtype, 0
    return a


def group_launch(outlined_name, ins, outs, act=("none",), pad=0, n_heads=0, eps=0.0, scale=0.0,
                 stream=None, res_arg=0, stride=1):
    """npu_group_launch: runs the outlined group(s) `outlined_name` ('+'-joined
    for a chain) on its arguments in the outlined function's order: ``ins``
    are tensors, Empty placeholders and the fill value (a float); ``outs`` the
    result tensors.  ``res_arg``: the index in ``ins`` of a conv group's
    residual operand (0: none named)."""
    keep = []
    ia = (_lib.NpuArg * max(len(ins), 1))(*[_group_arg(x, keep) for x in ins])
    oa = (_lib.NpuArg * max(len(outs), 1))(*[_group_arg(x, keep) for x in outs])
    at = _lib.NpuGroupAttrs()
    for i, a in enumerate(act):
        at.act[i] = ACT[a]
    at.pad, at.n_heads, at.eps, at.scale = int(pad), int(n_heads), float(eps), float(scale)
    at.res_arg, at.stride = int(res_arg), int(stride)
    st = _lib.lib().npu_group_launch(outlined_name.encode(), C.byref(at), ia, len(ins), oa,
                                     len(outs), _stream(stream))
    _check(st, f"npu_group_launch({outlined_name})")
    return outs


def llama_layer(p, bufs, n_heads, eps=1e-5, stream=None):
    """One decoder layer as its five groups.  ``p``: x, g1, g2, wq, wk, wv, wo,
    wg, wu, wd, cos_t, sin_t; ``bufs``: Q, K, V, A, h, act, out (caller-owned)."""
    fused_llama_qkv_rope(p["x"], p["g1"], p["wq"], p["wk"], p["wv"], p["cos_t"], p["sin_t"],
                         bufs["Q"], bufs["K"], bufs["V"], eps, stream)
    dh = p["x"].shape[1] // n_heads
    fused_llama_attention(bufs["Q"], bufs["K"], bufs["V"], bufs["A"], n_heads, dh ** -0.5, stream)
    fused_llama_matmul_residual(bufs["A"], p["wo"], p["x"], bufs["h"], stream)
    fused_llama_rmsnorm_swiglu(bufs["h"], p["g2"], p["wg"], p["wu"], bufs["act"], eps, stream)
    fused_llama_matmul_residual(bufs["act"], p["wd"], bufs["h"], bufs["out"], stream)
    return bufs["out"]
