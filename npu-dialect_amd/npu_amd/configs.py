"""The fused-block workloads: shapes, seeded inputs, algorithmic work, GPU launch.

Each workload is one fused group (or a chain of groups for the decoder
layer) at the sizes of one configuration.  ``flops`` and ``bytes`` are the
algorithmic figures: 2 x MACs of the contractions plus one op per output for
the epilogue where stated, and the compulsory HBM bytes of the fused block
(external inputs read once, outputs written once, intermediates excluded).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Callable

import numpy as np

from . import groups
from . import inputs as rng

# MI355X published peaks (dense).
PEAK = {
    "hbm": 8.0e12,          # B/s
    "f32": 157.3e12,        # FLOP/s (vector = matrix)
    "bf16": 2.5166e15,
    "i8": 5.033e15,
}


@dataclass
class Workload:
    name: str
    config: int
    dtype: str
    flops: int
    bytes: int
    make_inputs: Callable[[], dict]
    # (dev_inputs: dict[str, Tensor]) -> dict[str, Tensor] of empty outputs
    make_outputs: Callable[[dict], dict]
    # (dev_inputs, dev_outputs, stream) -> None ; issues the fused launches
    run: Callable[[dict, dict, object], None]
    desc: str = ""
    units: int = 1          # images / sequences per step (throughput unit)
    unit_name: str = "images"
    meta: dict = field(default_factory=dict)

    @property
    def bound(self) -> str:
        """'hbm' or 'mfma': which roofline term is larger at peak."""
        t_mem = self.bytes / PEAK["hbm"]
        t_cmp = self.flops / PEAK[self.peak_key]
        return "hbm" if t_mem >= t_cmp else "mfma"

    @property
    def peak_key(self) -> str:
        return {"f32": "f32", "bf16": "bf16", "i8": "i8"}[self.dtype]

    def floor_s(self) -> float:
        return max(self.bytes / PEAK["hbm"], self.flops / PEAK[self.peak_key])

    def roofline(self, seconds: float) -> dict:
        if self.bound == "hbm":
            achieved = self.bytes / seconds
            return {"bound": "hbm", "achieved": achieved / 1e9, "peak": PEAK["hbm"] / 1e9,
                    "unit": "GB/s", "frac": achieved / PEAK["hbm"]}
        achieved = self.flops / seconds
        return {"bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK[self.peak_key] / 1e12,
                "unit": "TFLOP/s", "frac": achieved / PEAK[self.peak_key]}


def _to_dev(arrs: dict) -> dict:
    import torch
    out = {}
    for k, v in arrs.items():
        if v is None:
            out[k] = None
        elif v.dtype == np.uint16:
            out[k] = torch.from_numpy(v.view(np.int16)).view(torch.bfloat16).cuda()
        else:
            out[k] = torch.from_numpy(np.ascontiguousarray(v)).cuda()
    return out


def to_device(arrs: dict) -> dict:
    return _to_dev(arrs)


def to_host(t) -> np.ndarray:
    import torch
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


# ------------------------------------------------------------------ C1
def matmul_bias_relu(M=256, K=512, N=256, seed=rng.SEED_BASE + 1) -> Workload:
    def make_inputs():
        return {
            "A": rng.uniform(seed, 0, (M, K), -1.0, 1.0),
            "B": rng.uniform(seed, 1, (K, N), -1.0, 1.0),
            "bias": rng.uniform(seed, 2, (N,), -1.0, 1.0),
        }

    def make_outputs(d):
        import torch
        return {"out": torch.empty((M, N), dtype=torch.float32, device="cuda")}

    def run(d, o, stream):
        groups.fused_matmul_bias_act(d["A"], d["B"], d["bias"], o["out"], "relu", stream)

    return Workload(
        name=f"matmul_bias_relu_f32_{M}x{K}x{N}", config=1, dtype="f32",
        flops=2 * M * N * K + 2 * M * N, bytes=4 * (M * K + K * N + N + M * N),
        make_inputs=make_inputs, make_outputs=make_outputs, run=run,
        desc=f"fill->matmul->bias+ReLU, A[{M}x{K}] B[{K}x{N}] f32", units=1, unit_name="blocks",
        meta={"M": M, "K": K, "N": N})


# ------------------------------------------------------------------ C2
def conv3x3_bias_relu(N=1, dtype="f32", H=56, W=56, C=64, F=64,
                      seed=rng.SEED_BASE + 2) -> Workload:
    KH = KW = 3
    esz = 4 if dtype == "f32" else 2

    def make_inputs():
        x = rng.uniform(seed, 0, (N, H, W, C), 0.0, 1.0)
        w = rng.normal(seed, 1, (F, KH, KW, C), 0.0, math.sqrt(2.0 / (KH * KW * C)))
        b = rng.uniform(seed, 2, (F,), -0.1, 0.1)
        if dtype == "bf16":
            x, w = rng.to_bf16_bits(x), rng.to_bf16_bits(w)
        return {"x": x, "w": w, "bias": b}

    def make_outputs(d):
        import torch
        tdt = torch.float32 if dtype == "f32" else torch.bfloat16
        return {"out": torch.empty((N, H, W, F), dtype=tdt, device="cuda")}

    def run(d, o, stream):
        groups.fused_conv2d_nhwc_bias_act(d["x"], d["w"], d["bias"], o["out"], 1, "relu", stream)

    P = N * H * W
    return Workload(
        name=f"conv3x3_bias_relu_{dtype}_n{N}", config=2, dtype=dtype,
        flops=2 * P * F * KH * KW * C + 2 * P * F,
        bytes=esz * (P * C + P * F + F * KH * KW * C) + 4 * F,
        make_inputs=make_inputs, make_outputs=make_outputs, run=run,
        desc=f"pad->conv2d 3x3 NHWC {N}x{H}x{W}x{C} -> {F} +bias+ReLU ({dtype})", units=N,
        meta={"N": N, "H": H, "W": W, "C": C, "F": F})


def all_workloads() -> list:
    """Every configuration this backend runs, in configuration order."""
    return [
        matmul_bias_relu(),
        conv3x3_bias_relu(1, "f32"), conv3x3_bias_relu(32, "f32"),
        conv3x3_bias_relu(1, "bf16"), conv3x3_bias_relu(32, "bf16"),
    ]


HEADLINE = "conv3x3_bias_relu_f32_n32"


def by_name(name: str) -> Workload:
    for w in all_workloads():
        if w.name == name:
            return w
    raise KeyError(name)
