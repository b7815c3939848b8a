"""Oracle results and error-bound magnitudes for each workload's inputs.

TEST INFRASTRUCTURE ONLY (see oracle.py).  ``reference(name, inputs)`` runs
the unfused CPU restatement of the workload's linalg chain and returns
``{output_name: (expected, mag)}`` where ``mag`` is the chain evaluated on
absolute values (the scale of the per-element error bound) or None for
integer outputs that must match bit for bit.
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


def run_oracle(workload_name: str, inp: dict, images=None) -> dict:
    """Only the oracle's outputs (what the CPU baseline times)."""
    sel = (lambda a: a) if images is None else (lambda a: np.ascontiguousarray(a[list(images)]))
    if workload_name.startswith("matmul_bias_relu"):
        return {"out": oracle.block_matmul_bias_act(inp["A"], inp["B"], inp["bias"], "relu")}
    if workload_name.startswith("conv3x3_bias_relu"):
        return {"out": oracle.block_conv_bias_act(sel(inp["x"]), inp["w"], inp["bias"], 1, "relu")}
    raise KeyError(workload_name)


def reference(workload_name: str, inp: dict, images=None) -> dict:
    """Expected outputs of a named workload; ``images`` restricts batched
    workloads to a subset of batch indices (each image is independent)."""
    sel = (lambda a: a) if images is None else (lambda a: np.ascontiguousarray(a[list(images)]))
    if workload_name.startswith("matmul_bias_relu"):
        return {"out": matmul_bias_act(inp["A"], inp["B"], inp["bias"], "relu")}
    if workload_name.startswith("conv3x3_bias_relu"):
        return {"out": conv_bias_act(sel(inp["x"]), inp["w"], inp["bias"], 1, "relu")}
    raise KeyError(workload_name)
