"""ctypes front end of the CPU restatement (libnpu_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the HIP product path.  Only the
tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module.  It restates the reference's CPU
execution of lowered linalg (tools/harness/e2e_verify.py:232-251); see
npu_oracle.h for the per-op citations and parity status.

All arrays are numpy, C-contiguous.  bf16 tensors are ``np.uint16`` bit
patterns.  Functions allocate and return their outputs.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libnpu_oracle.so")
_OMP_PATH = os.path.join(_HERE, "libnpu_oracle_omp.so")
_libs = {}
_threaded = False

_I64 = C.c_int64
_F32 = C.c_float
_PTR = C.c_void_p


def build() -> None:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


def lib():
    path = _OMP_PATH if _threaded else _LIB_PATH
    if path not in _libs:
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run make -C oracle)")
        _libs[path] = C.CDLL(path)
    return _libs[path]


class threaded:
    """Context manager: the oracle calls inside it run the OpenMP build
    (outer parallel loops over OMP_NUM_THREADS threads; same results)."""

    def __enter__(self):
        global _threaded
        self._prev, _threaded = _threaded, True
        return self

    def __exit__(self, *exc):
        global _threaded
        _threaded = self._prev
        return False


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return C.c_void_p(a.ctypes.data)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u16(a):
    a = np.ascontiguousarray(a)
    assert a.dtype == np.uint16, "bf16 tensors are carried as uint16 bit patterns"
    return a


def _i8(a):
    return np.ascontiguousarray(a, dtype=np.int8)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _call(name, *args):
    fn = getattr(lib(), name)
    conv = []
    for a in args:
        if isinstance(a, np.ndarray):
            conv.append(_p(a))
        elif isinstance(a, float):
            conv.append(_F32(a))
        elif isinstance(a, (int, np.integer)):
            conv.append(_I64(int(a)))
        elif a is None:
            conv.append(C.c_void_p(0))
        else:
            raise TypeError(type(a))
    fn.restype = None
    fn(*conv)


# ---------------------------------------------------------------- elementary
def matmul(A, B, C0=None):
    """linalg.matmul into a zero (or given) init: C += A@B, loops m,n,k."""
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    Cm = np.zeros((M, N), np.float32) if C0 is None else _f32(C0).copy()
    _call("orc_matmul_f32", A, K, B, N, Cm, N, M, N, K)
    return Cm


def matmul_tiled_m(A, B, tile_m):
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    N = B.shape[1]
    Cm = np.zeros((M, N), np.float32)
    _call("orc_matmul_tiled_m_f32", A, B, Cm, M, N, K, tile_m)
    return Cm


def matmul_bf16(A, B):
    A, B = _u16(A), _u16(B)
    M, K = A.shape
    N = B.shape[1]
    Cm = np.zeros((M, N), np.float32)
    _call("orc_matmul_bf16_f32", A, K, B, N, Cm, N, M, N, K)
    return Cm


def batch_matmul(A, B):
    A, B = _f32(A), _f32(B)
    Bt, M, K = A.shape
    N = B.shape[2]
    Cm = np.zeros((Bt, M, N), np.float32)
    _call("orc_batch_matmul_f32", A, B, Cm, Bt, M, N, K)
    return Cm


def relu(x):
    x = _f32(x)
    o = np.empty_like(x)
    _call("orc_relu_f32", x, o, x.size)
    return o


def relu6(x):
    x = _f32(x)
    o = np.empty_like(x)
    _call("orc_relu6_f32", x, o, x.size)
    return o


def add(a, b):
    a, b = _f32(a), _f32(b)
    o = np.empty_like(a)
    _call("orc_add_f32", a, b, o, a.size)
    return o


def bias_add(x, bias):
    x, bias = _f32(x), _f32(bias)
    o = np.empty_like(x)
    _call("orc_bias_add_f32", x, bias, o, x.size // bias.size, bias.size)
    return o


def silu_mul(g, u):
    g, u = _f32(g), _f32(u)
    o = np.empty_like(g)
    _call("orc_silu_mul_f32", g, u, o, g.size)
    return o


def pad_nchw(x, pads, value=0.0):
    x = _f32(x)
    N, Cc, H, W = x.shape
    pt, pb, pl, pr = pads
    o = np.empty((N, Cc, H + pt + pb, W + pl + pr), np.float32)
    _call("orc_pad_nchw_f32", x, o, N, Cc, H, W, pt, pb, pl, pr, float(value))
    return o


def pad_nhwc(x, pads, value=0.0):
    N, H, W, Cc = x.shape
    pt, pb, pl, pr = pads
    if x.dtype == np.uint16:
        x = _u16(x)
        o = np.empty((N, H + pt + pb, W + pl + pr, Cc), np.uint16)
        _call("orc_pad_nhwc_u16", x, o, N, H, W, Cc, pt, pb, pl, pr)
    elif x.dtype == np.int8:
        x = _i8(x)
        o = np.empty((N, H + pt + pb, W + pl + pr, Cc), np.int8)
        _call("orc_pad_nhwc_i8", x, o, N, H, W, Cc, pt, pb, pl, pr)
    else:
        x = _f32(x)
        o = np.empty((N, H + pt + pb, W + pl + pr, Cc), np.float32)
        _call("orc_pad_nhwc_f32", x, o, N, H, W, Cc, pt, pb, pl, pr, float(value))
    return o


def conv2d_nchw_fchw(xp, w, stride=(1, 1)):
    xp, w = _f32(xp), _f32(w)
    N, Cc, Hp, Wp = xp.shape
    F, C2, KH, KW = w.shape
    assert Cc == C2
    Ho, Wo = (Hp - KH) // stride[0] + 1, (Wp - KW) // stride[1] + 1
    o = np.zeros((N, F, Ho, Wo), np.float32)
    _call("orc_conv2d_nchw_fchw_f32", xp, w, o, N, Cc, Hp, Wp, F, KH, KW, stride[0], stride[1])
    return o


def conv2d_nhwc_fhwc(xp, w, stride=(1, 1)):
    """Pre-padded NHWC input, FHWC filter.  f32, bf16 (-> f32) or i8 (-> i32)."""
    N, Hp, Wp, Cc = xp.shape
    F, KH, KW, C2 = w.shape
    assert Cc == C2
    Ho, Wo = (Hp - KH) // stride[0] + 1, (Wp - KW) // stride[1] + 1
    if xp.dtype == np.int8:
        o = np.zeros((N, Ho, Wo, F), np.int32)
        _call("orc_conv2d_nhwc_fhwc_i8_i32", _i8(xp), _i8(w), o, N, Hp, Wp, Cc, F, KH, KW,
              stride[0], stride[1])
    elif xp.dtype == np.uint16:
        o = np.zeros((N, Ho, Wo, F), np.float32)
        _call("orc_conv2d_nhwc_fhwc_bf16_f32", _u16(xp), _u16(w), o, N, Hp, Wp, Cc, F, KH, KW,
              stride[0], stride[1])
    else:
        o = np.zeros((N, Ho, Wo, F), np.float32)
        _call("orc_conv2d_nhwc_fhwc_f32", _f32(xp), _f32(w), o, N, Hp, Wp, Cc, F, KH, KW,
              stride[0], stride[1])
    return o


def depthwise_conv2d_nhwc_hwc(xp, w, stride=(1, 1)):
    xp, w = _f32(xp), _f32(w)
    N, Hp, Wp, Cc = xp.shape
    KH, KW, C2 = w.shape
    assert Cc == C2
    Ho, Wo = (Hp - KH) // stride[0] + 1, (Wp - KW) // stride[1] + 1
    o = np.zeros((N, Ho, Wo, Cc), np.float32)
    _call("orc_depthwise_conv2d_nhwc_hwc_f32", xp, w, o, N, Hp, Wp, Cc, KH, KW, stride[0],
          stride[1])
    return o


def trunc_bf16(x):
    x = _f32(x)
    o = np.empty(x.shape, np.uint16)
    _call("orc_trunc_f32_bf16", x, o, x.size)
    return o


def ext_bf16(x):
    x = _u16(x)
    o = np.empty(x.shape, np.float32)
    _call("orc_ext_bf16_f32", x, o, x.size)
    return o


def apply_scale(acc, mult, shift):
    acc, mult, shift = _i32(acc), _i32(mult), _i32(shift)
    o = np.empty_like(acc)
    cols = mult.size
    _call("orc_apply_scale_i32", acc, mult, shift, o, acc.size // cols, cols)
    return o


def clamp_i8(x, lo, hi):
    x = _i32(x)
    o = np.empty(x.shape, np.int8)
    fn = lib().orc_clamp_i32_i8
    fn.restype = None
    fn(_p(x), _p(o), _I64(x.size), C.c_int32(lo), C.c_int32(hi))
    return o


def rmsnorm(x, g, eps):
    x, g = _f32(x), _f32(g)
    o = np.empty_like(x)
    _call("orc_rmsnorm_f32", x, g, o, x.size // g.size, g.size, float(eps))
    return o


def rope(x, cos_t, sin_t, H):
    x, cos_t, sin_t = _f32(x), _f32(cos_t), _f32(sin_t)
    S, D = x.shape
    o = np.empty_like(x)
    _call("orc_rope_f32", x, cos_t, sin_t, o, S, H, D // H)
    return o


def causal_softmax(s):
    s = _f32(s).copy()
    rows, cols = s.shape
    _call("orc_causal_softmax_f32", s, rows, cols)
    return s


# ---------------------------------------------------------------- blocks
ACT = {"none": 0, "relu": 1, "relu6": 2}


def block_matmul_bias_act(A, B, bias, act="relu"):
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    N = B.shape[1]
    o = np.empty((M, N), np.float32)
    _call("orc_block_matmul_bias_act_f32", A, B, None if bias is None else _f32(bias), o, M, N,
          K, ACT[act])
    return o


def block_conv_bias_act(x, w, bias, pad=1, act="relu"):
    N, H, W, Cc = x.shape
    F, KH, KW, _ = w.shape
    Ho, Wo = H + 2 * pad - KH + 1, W + 2 * pad - KW + 1
    b = None if bias is None else _f32(bias)
    if x.dtype == np.uint16:
        o = np.empty((N, Ho, Wo, F), np.uint16)
        _call("orc_block_conv_bias_act_bf16", _u16(x), _u16(w), b, o, N, H, W, Cc, F, KH, KW,
              pad, ACT[act])
    else:
        o = np.empty((N, Ho, Wo, F), np.float32)
        _call("orc_block_conv_bias_act_f32", _f32(x), _f32(w), b, o, N, H, W, Cc, F, KH, KW,
              pad, ACT[act])
    return o


def block_irb(x, we, wdw, wp):
    x, we, wdw, wp = _f32(x), _f32(we), _f32(wdw), _f32(wp)
    N, H, W, Cc = x.shape
    E = we.shape[0]
    o = np.empty_like(x)
    _call("orc_block_irb_f32", x, we, wdw, wp, o, N, H, W, Cc, E)
    return o


def block_qbottleneck(x, w1, w2, w3, m1, s1, m2, s2, m3, s3):
    x = _i8(x)
    N, H, W, Cc = x.shape
    M1 = w1.shape[0]
    o = np.empty_like(x)
    _call("orc_block_qbottleneck_i8", x, _i8(w1), _i8(w2), _i8(w3), _i32(m1), _i32(s1), _i32(m2),
          _i32(s2), _i32(m3), _i32(s3), o, N, H, W, Cc, M1)
    return o


def llama_qkv(x, g1, wq, wk, wv, cos_t, sin_t, H, eps):
    S, D = x.shape
    Q = np.empty((S, D), np.uint16)
    K = np.empty((S, D), np.uint16)
    V = np.empty((S, D), np.uint16)
    _call("orc_llama_qkv_bf16", _u16(x), _f32(g1), _u16(wq), _u16(wk), _u16(wv), _f32(cos_t),
          _f32(sin_t), Q, K, V, S, D, H, float(eps))
    return Q, K, V


def llama_attention(Q, K, V, H, scale):
    S, D = Q.shape
    A = np.empty((S, D), np.uint16)
    _call("orc_llama_attention_bf16", _u16(Q), _u16(K), _u16(V), A, S, H, D // H, float(scale))
    return A


def llama_matmul_residual(a, w, res):
    S, Kd = a.shape
    N = w.shape[1]
    o = np.empty((S, N), np.uint16)
    _call("orc_llama_matmul_residual_bf16", _u16(a), _u16(w), _u16(res), o, S, N, Kd)
    return o


def llama_swiglu(h, g2, wg, wu, eps):
    S, D = h.shape
    F = wg.shape[1]
    o = np.empty((S, F), np.uint16)
    _call("orc_llama_swiglu_bf16", _u16(h), _f32(g2), _u16(wg), _u16(wu), o, S, D, F, float(eps))
    return o


def block_llama_layer(x, g1, g2, wq, wk, wv, wo, wg, wu, wd, cos_t, sin_t, H, eps):
    S, D = x.shape
    F = wg.shape[1]
    h = np.empty((S, D), np.uint16)
    o = np.empty((S, D), np.uint16)
    _call("orc_block_llama_layer_bf16", _u16(x), _f32(g1), _f32(g2), _u16(wq), _u16(wk),
          _u16(wv), _u16(wo), _u16(wg), _u16(wu), _u16(wd), _f32(cos_t), _f32(sin_t), h, o, S, D,
          H, F, float(eps))
    return h, o
