"""npu_amd -- MI355X (gfx950) execution backend for NPU-Dialect's fused tile groups.

Host-side Python mirror of the C-ABI in include/npu_amd.h.  The kernels are
hand-written HIP in ../csrc, built into libnpu_amd.so next to this file.
"""
from ._lib import build, lib  # noqa: F401
from .groups import NpuError, fused_conv2d_nhwc_bias_act, fused_matmul_bias_act  # noqa: F401

__all__ = ["build", "lib", "NpuError", "fused_matmul_bias_act", "fused_conv2d_nhwc_bias_act"]
