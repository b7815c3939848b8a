"""Loads libnpu_amd.so (the HIP kernels and their extern "C" ABI) with ctypes.

The library is built in-tree by ``make -C npu-dialect_amd``; there is no
fallback.  If the shared object is missing or lacks a symbol the headers
declare, loading fails with an error naming the file, so a GPU run can never
silently execute anything but the HIP path.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libnpu_amd.so")
SRC_DIR = os.path.dirname(PKG_DIR)

# Every extern "C" symbol of include/npu_amd.h, with its ctypes signature.
_I32, _I64, _P = C.c_int32, C.c_int64, C.c_void_p


class NpuMemref(C.Structure):
    """npu_memref: {allocated, aligned, offset, sizes[4], strides[4], rank, dtype}."""

    _fields_ = [
        ("allocated", C.c_void_p),
        ("aligned", C.c_void_p),
        ("offset", C.c_int64),
        ("sizes", C.c_int64 * 4),
        ("strides", C.c_int64 * 4),
        ("rank", C.c_int32),
        ("dtype", C.c_int32),
    ]


_MR = C.POINTER(NpuMemref)


class NpuLaunchPlan(C.Structure):
    """npu_launch_plan: per-tile work of one kernel launch (launch-model input)."""

    _fields_ = [
        ("kernel", C.c_char * 48),
        ("grid", C.c_int32),
        ("wg_per_cu", C.c_int32),
        ("tiles", C.c_int32),
        ("load_phases", C.c_int32),
        ("mfma_bits", C.c_int32),
        ("unit_waves", C.c_int32),
        ("tile_macs", C.c_double),
        ("tile_valu", C.c_double),
        ("tile_lds_bytes", C.c_double),
        ("tile_load_bytes", C.c_double),
        ("tile_store_bytes", C.c_double),
        ("wg_setup_bytes", C.c_double),
        ("hbm_bytes", C.c_double),
        ("wg_setup_valu", C.c_double),
    ]

def strided_memref_type(rank: int):
    """MLIR's StridedMemRefType<T, rank> layout: {allocated, aligned, offset,
    sizes[rank], strides[rank]} (include/npu_amd.h NPU_STRIDED_MEMREF)."""
    class StridedMemref(C.Structure):
        _fields_ = [("allocated", C.c_void_p), ("aligned", C.c_void_p), ("offset", C.c_int64),
                    ("sizes", C.c_int64 * rank), ("strides", C.c_int64 * rank)]
    return StridedMemref


class NpuArg(C.Structure):
    """npu_arg: MLIR's UnrankedMemRefType {rank, descriptor}, then the element
    type and, for a scalar argument, its value."""

    _fields_ = [
        ("rank", C.c_int64),
        ("descriptor", C.c_void_p),
        ("dtype", C.c_int32),
        ("kind", C.c_int32),
        ("scalar", C.c_double),
    ]


class NpuGroupAttrs(C.Structure):
    """npu_group_attrs: per-chain activations, folded pad, heads, eps, scale,
    the residual operand's argument index, the conv stride."""

    _fields_ = [
        ("act", C.c_int32 * 16),
        ("pad", C.c_int32),
        ("n_heads", C.c_int32),
        ("eps", C.c_float),
        ("scale", C.c_float),
        ("res_arg", C.c_int32),
        ("stride", C.c_int32),
    ]


class NpuTilePlan(C.Structure):
    """npu_tile_plan: the temporal tile and each SRAM buffer's LDS offset."""

    _fields_ = [
        ("tm", C.c_int32), ("tn", C.c_int32), ("tk", C.c_int32), ("lds_bytes", C.c_int32),
        ("off_a", C.c_int64), ("off_a_pong", C.c_int64),
        ("off_b", C.c_int64), ("off_b_pong", C.c_int64),
        ("off_bias", C.c_int64), ("off_c", C.c_int64), ("off_y", C.c_int64),
    ]


class NpuConvTilePlan(C.Structure):
    """npu_conv_tile_plan: the output-channel tile and each SRAM buffer's LDS
    offset (ping, pong, prefetch region; -1 where the plan has none)."""

    _fields_ = [
        ("tco", C.c_int32), ("lds_bytes", C.c_int32),
        ("off_in", C.c_int64), ("off_in_pong", C.c_int64), ("off_in_prefetch", C.c_int64),
        ("off_w", C.c_int64), ("off_w_pong", C.c_int64), ("off_w_prefetch", C.c_int64),
        ("off_bias", C.c_int64), ("off_bias_pong", C.c_int64), ("off_bias_prefetch", C.c_int64),
        ("off_c", C.c_int64), ("off_y", C.c_int64),
    ]


_ARG = C.POINTER(NpuArg)

SIGNATURES = {
    "npu_version": (C.c_char_p, []),
    "npu_last_error": (C.c_char_p, []),
    "npu_status_string": (C.c_char_p, [_I32]),
    "npu_device_count": (_I32, []),
    "fused_matmul_bias_act": (_I32, [_MR, _MR, _MR, _MR, _I32, _P]),
    "npu_planned_matmul_bias_act": (_I32, [_MR, _MR, _MR, _MR, _I32, C.POINTER(NpuTilePlan), _P,
                                           _P]),
    "npu_planned_conv2d_nchw_bias_act": (_I32, [_MR, _MR, _MR, _MR, _I32,
                                                C.POINTER(NpuConvTilePlan), _P, _P]),
    "fused_conv2d_nhwc_bias_act": (_I32, [_MR, _MR, _MR, _MR, _I32, _I32, _P]),
    "fused_conv2d_nhwc_bias_res_act": (_I32, [_MR, _MR, _MR, _MR, _MR, _I32, _I32, _P]),
    "fused_conv2d_nchw_bias_act": (_I32, [_MR, _MR, _MR, _MR, _I32, _I32, _I32, _P]),
    "fused_conv2d_nchw_bias_res_act": (_I32, [_MR, _MR, _MR, _MR, _MR, _I32, _I32, _I32, _P]),
    "fused_qbottleneck_i8": (_I32, [_MR] * 11 + [_P]),
    "fused_irb_f32": (_I32, [_MR] * 5 + [_P]),
    "fused_llama_qkv_rope": (_I32, [_MR] * 10 + [C.c_float, _P]),
    "fused_llama_attention": (_I32, [_MR] * 4 + [_I32, C.c_float, _P]),
    "fused_llama_matmul_residual": (_I32, [_MR] * 4 + [_P]),
    "fused_llama_rmsnorm_swiglu": (_I32, [_MR] * 5 + [C.c_float, _P]),
    "npu_group_launch": (_I32, [C.c_char_p, C.POINTER(NpuGroupAttrs), _ARG, _I32, _ARG, _I32,
                                _P]),
    "npu_last_launch_plans": (_I32, [C.POINTER(NpuLaunchPlan), _I32]),
}

_lib = None


def build() -> None:
    """Compile every HIP source for gfx950 into libnpu_amd.so (always rebuilds)."""
    subprocess.run(["make", "-s", "-B", "-j8", "-C", SRC_DIR], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libnpu_amd.so not found at {LIB_PATH}: build it with `make -C {SRC_DIR}` "
                "(the HIP path has no fallback)")
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)  # AttributeError names a missing export
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_launch_plans():
    """Launch plans of this thread's most recent fused_* call (a list of NpuLaunchPlan)."""
    n = lib().npu_last_launch_plans(None, 0)
    arr = (NpuLaunchPlan * max(n, 1))()
    lib().npu_last_launch_plans(arr, n)
    return [arr[i] for i in range(n)]
