"""Python mirror of the fused-group entry points (include/npu_amd.h).

Each function takes torch tensors that already live on the GPU, builds the
npu_memref descriptors and calls the extern "C" entry point on the current
torch stream (or the given one).  A non-OK status raises NpuError with the
library's own message; nothing falls back to another implementation.

The group names follow the op chains the reference's outliner groups
(lib/Transforms/OutlineFusedGroupsPass.cpp:259-263): see ``OUTLINED_NAMES``.
"""
from __future__ import annotations

from . import _lib
from .memref import absent, from_tensor, ref

ACT = {"none": 0, "relu": 1, "relu6": 2}

# Outlined-function name (without the _<idx> suffix) -> entry point.  The
# short op names follow OutlineFusedGroupsPass.cpp:69-82; ops the reference
# has no short name for use ours (conv2d_nhwc, dwconv2d, pad).
OUTLINED_NAMES = {
    "fused_fill_matmul_generic": "fused_matmul_bias_act",
    "fused_pad_fill_conv2d_nhwc_generic": "fused_conv2d_nhwc_bias_act",
}


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


def _check(status, where):
    if status != 0:
        raise NpuError(status, where)


def _opt(t):
    return absent() if t is None else from_tensor(t)


def fused_matmul_bias_act(A, B, bias, out, act="relu", stream=None):
    """out = act(A @ B + bias); f32 [M,K] @ [K,N] (+ [N])."""
    mA, mB, mb, mo = from_tensor(A), from_tensor(B), _opt(bias), from_tensor(out)
    st = _lib.lib().fused_matmul_bias_act(ref(mA), ref(mB), ref(mb), ref(mo), ACT[act],
                                          _stream(stream))
    _check(st, "fused_matmul_bias_act")
    return out


def fused_conv2d_nhwc_bias_act(x, w, bias, out, pad=1, act="relu", stream=None):
    """out = act(conv_2d_nhwc_fhwc(pad(x), w) + bias); f32 or bf16."""
    mx, mw, mb, mo = from_tensor(x), from_tensor(w), _opt(bias), from_tensor(out)
    st = _lib.lib().fused_conv2d_nhwc_bias_act(ref(mx), ref(mw), ref(mb), ref(mo), int(pad),
                                               ACT[act], _stream(stream))
    _check(st, "fused_conv2d_nhwc_bias_act")
    return out
