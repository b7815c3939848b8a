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
    # The matrix pipe the launch runs its contractions on and the work it
    # does there per algorithmic flop: an f32 block that the GPU computes as
    # three-part bf16 splits runs six bf16 products per f32 product on the
    # bf16 pipe (mfma_key "bf16", mfma_factor 6).
    mfma_key: str = ""
    mfma_factor: int = 1

    @property
    def bound(self) -> str:
        """'hbm' or 'mfma': which roofline term is larger at peak."""
        t_mem = self.bytes / PEAK["hbm"]
        t_cmp = self.mfma_flops / PEAK[self.peak_key]
        return "hbm" if t_mem >= t_cmp else "mfma"

    @property
    def peak_key(self) -> str:
        return self.mfma_key or {"f32": "f32", "bf16": "bf16", "i8": "i8"}[self.dtype]

    @property
    def mfma_flops(self) -> int:
        """Matrix-pipe work of one launch (flops of the pipe's own type)."""
        return self.flops * self.mfma_factor

    def floor_s(self) -> float:
        return max(self.bytes / PEAK["hbm"], self.mfma_flops / PEAK[self.peak_key])

    def roofline(self, seconds: float) -> dict:
        if self.bound == "hbm":
            achieved = self.bytes / seconds
            return {"bound": "hbm", "achieved": achieved / 1e9, "peak": PEAK["hbm"] / 1e9,
                    "unit": "GB/s", "frac": achieved / PEAK["hbm"]}
        achieved = self.mfma_flops / seconds
        out = {"bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK[self.peak_key] / 1e12,
               "unit": "TFLOP/s", "frac": achieved / PEAK[self.peak_key]}
        if self.mfma_factor != 1:
            out["pipe"] = f"{self.peak_key} ({self.mfma_factor} products per {self.dtype} product)"
            out["algorithmic_tflops"] = self.flops / seconds / 1e12
        return out


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
    # the f32 persistent launch (>= 48 row pairs, F a multiple of 64, 32 or
    # 64 channels) multiplies on the bf16 pipe, six products per f32 product
    on_bf16 = dtype == "f32" and N * ((H + 1) // 2) >= 48 and F % 64 == 0 and C in (32, 64) and W <= 64
    return Workload(
        name=f"conv3x3_bias_relu_{dtype}_n{N}", config=2, dtype=dtype,
        flops=2 * P * F * KH * KW * C + 2 * P * F,
        bytes=esz * (P * C + P * F + F * KH * KW * C) + 4 * F,
        make_inputs=make_inputs, make_outputs=make_outputs, run=run,
        desc=f"pad->conv2d 3x3 NHWC {N}x{H}x{W}x{C} -> {F} +bias+ReLU ({dtype})", units=N,
        meta={"N": N, "H": H, "W": W, "C": C, "F": F},
        mfma_key="bf16" if on_bf16 else "", mfma_factor=6 if on_bf16 else 1)


# ------------------------------------------------------------------ C3
def irb(N=1, H=56, W=56, C=24, E=144, seed=rng.SEED_BASE + 3) -> Workload:
    def make_inputs():
        return {
            "x": rng.uniform(seed, 0, (N, H, W, C), 0.0, 1.0),
            "we": rng.normal(seed, 1, (E, C), 0.0, math.sqrt(2.0 / C)),
            "wdw": rng.normal(seed, 2, (3, 3, E), 0.0, math.sqrt(2.0 / 9)),
            "wp": rng.normal(seed, 3, (C, E), 0.0, math.sqrt(2.0 / E)),
        }

    def make_outputs(d):
        import torch
        return {"out": torch.empty((N, H, W, C), dtype=torch.float32, device="cuda")}

    def run(d, o, stream):
        groups.fused_irb_f32(d["x"], d["we"], d["wdw"], d["wp"], o["out"], stream)

    P = N * H * W
    return Workload(
        name=f"mbv2_irb_f32_n{N}", config=3, dtype="f32",
        flops=2 * P * (C * E + 9 * E + E * C),
        bytes=4 * (2 * P * C + E * C + 9 * E + C * E),
        make_inputs=make_inputs, make_outputs=make_outputs, run=run,
        desc=f"MobileNetV2 IRB 1x1 {C}->{E} ReLU6, dw3x3 ReLU6, 1x1 {E}->{C}, +x; NHWC "
             f"{N}x{H}x{W} f32", units=N, meta={"N": N, "H": H, "W": W, "C": C, "E": E})


# ------------------------------------------------------------------ C4
def quant_multiplier(real):
    """Fixed-point (multiplier, shift) with real ~= m * 2^-shift, m in [2^30, 2^31)."""
    real = np.asarray(real, np.float64)
    frac, exp = np.frexp(real)                      # real = frac * 2^exp, frac in [0.5, 1)
    m = np.rint(frac * 2.0 ** 31).astype(np.int64)
    exp = exp + (m == 2 ** 31)
    m = np.where(m == 2 ** 31, 2 ** 30, m)
    shift = 31 - exp
    if np.any(shift < 2) or np.any(shift > 62):
        raise ValueError("requant scale out of the apply_scale range")
    return m.astype(np.int32), shift.astype(np.int32)


def requant_np(acc, m, s):
    acc = np.asarray(acc, np.int64)
    return (acc * m.astype(np.int64) + (np.int64(1) << (s.astype(np.int64) - 1))) >> s


def _quantize_per_channel(wf):
    flat = wf.reshape(wf.shape[0], -1).astype(np.float64)
    sc = np.abs(flat).max(1) / 127.0
    q = np.clip(np.rint(flat / sc[:, None]), -127, 127).astype(np.int8)
    return q.reshape(wf.shape), sc


def qbottleneck(N=32, H=56, W=56, C=256, M1=64, seed=rng.SEED_BASE + 4) -> Workload:
    """int8 ResNet-50 bottleneck.  Weights: He-normal floats quantized per
    output channel, symmetric, to [-127, 127].  Activations: int8 with zero
    point 0 and scale 1/127 for x and the output (so the residual adds
    directly).  Requant multipliers come from float scales calibrated once on
    image 0 (99.9th percentile of each post-ReLU activation mapped to 127)."""

    def make_inputs():
        x = rng.randint(seed, 0, (N, H, W, C), 0, 127).astype(np.int8)
        w1, sw1 = _quantize_per_channel(rng.normal(seed, 1, (M1, C), 0, math.sqrt(2 / C)))
        w2, sw2 = _quantize_per_channel(rng.normal(seed, 2, (M1, 3, 3, M1), 0,
                                                   math.sqrt(2 / (9 * M1))))
        w3, sw3 = _quantize_per_channel(rng.normal(seed, 3, (C, M1), 0, math.sqrt(2 / M1)))
        sx = 1.0 / 127
        x0 = x[0].astype(np.int64).reshape(-1, C)
        acc1 = x0 @ w1.astype(np.int64).T
        sy1 = np.percentile(np.maximum(acc1 * (sx * sw1), 0), 99.9) / 127
        m1, s1 = quant_multiplier(sx * sw1 / sy1)
        y1 = np.clip(requant_np(acc1, m1, s1), 0, 127).reshape(H, W, M1)
        y1p = np.pad(y1, ((1, 1), (1, 1), (0, 0)))
        cols = np.concatenate([y1p[kh:kh + H, kw:kw + W] for kh in range(3) for kw in range(3)],
                              -1).reshape(-1, 9 * M1)
        acc2 = cols @ w2.reshape(M1, -1).astype(np.int64).T
        sy2 = np.percentile(np.maximum(acc2 * (sy1 * sw2), 0), 99.9) / 127
        m2, s2 = quant_multiplier(sy1 * sw2 / sy2)
        m3, s3 = quant_multiplier(sy2 * sw3 / sx)
        return {"x": x, "w1": w1, "w2": w2, "w3": w3, "m1": m1, "s1": s1, "m2": m2, "s2": s2,
                "m3": m3, "s3": s3}

    def make_outputs(d):
        import torch
        return {"out": torch.empty((N, H, W, C), dtype=torch.int8, device="cuda")}

    def run(d, o, stream):
        groups.fused_qbottleneck_i8(d["x"], d["w1"], d["w2"], d["w3"], d["m1"], d["s1"],
                                    d["m2"], d["s2"], d["m3"], d["s3"], o["out"], stream)

    P = N * H * W
    wbytes = M1 * C + 9 * M1 * M1 + C * M1
    return Workload(
        name=f"qbottleneck_i8_n{N}", config=4, dtype="i8",
        flops=2 * P * (C * M1 + 9 * M1 * M1 + M1 * C),
        bytes=2 * P * C + wbytes + 4 * (4 * M1 + 2 * C),
        make_inputs=make_inputs, make_outputs=make_outputs, run=run,
        desc=f"int8 bottleneck 1x1 {C}->{M1}, 3x3 {M1}->{M1}, 1x1 {M1}->{C} + residual, "
             f"NHWC {N}x{H}x{W}", units=N, meta={"N": N, "H": H, "W": W, "C": C, "M1": M1})


# ------------------------------------------------------------------ C5
def rope_tables(S, Dh, theta=10000.0):
    """cos/sin of position * theta^(-2t/Dh), t < Dh/2, in float64 rounded to f32."""
    inv = theta ** (-np.arange(0, Dh, 2, dtype=np.float64) / Dh)
    ang = np.arange(S, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def llama_layer(S=512, D=512, H=8, F=1408, eps=1e-5, seed=rng.SEED_BASE + 5) -> Workload:
    """One Llama decoder layer, bf16: x ~ N(0,1), weights ~ N(0, 0.02), RMSNorm
    gains ~ U(0.5, 1.5) (f32), RoPE theta 10000, causal attention."""
    Dh = D // H

    def make_inputs():
        bf = lambda t, shape, sd: rng.to_bf16_bits(rng.normal(seed, t, shape, 0.0, sd))
        c, s = rope_tables(S, Dh)
        return {
            "x": bf(0, (S, D), 1.0),
            "wq": bf(1, (D, D), 0.02), "wk": bf(2, (D, D), 0.02), "wv": bf(3, (D, D), 0.02),
            "wo": bf(4, (D, D), 0.02), "wg": bf(5, (D, F), 0.02), "wu": bf(6, (D, F), 0.02),
            "wd": bf(7, (F, D), 0.02),
            "g1": rng.uniform(seed, 8, (D,), 0.5, 1.5), "g2": rng.uniform(seed, 9, (D,), 0.5, 1.5),
            "cos_t": c, "sin_t": s,
        }

    def make_outputs(d):
        import torch
        e = lambda *shape: torch.empty(shape, dtype=torch.bfloat16, device="cuda")
        return {"Q": e(S, D), "K": e(S, D), "V": e(S, D), "A": e(S, D), "h": e(S, D),
                "act": e(S, F), "out": e(S, D)}

    def run(d, o, stream):
        groups.llama_layer(d, o, H, eps, stream)

    pairs = S * (S + 1) // 2  # causal (query, key) pairs
    flops = 2 * S * D * 3 * D + 2 * H * Dh * pairs * 2 + 2 * S * D * D + 2 * S * D * 2 * F \
        + 2 * S * F * D
    wbytes = 2 * (4 * D * D + 3 * D * F)
    return Workload(
        name=f"llama_layer_bf16_s{S}", config=5, dtype="bf16", flops=flops,
        bytes=wbytes + 4 * 2 * D + 2 * 4 * S * (Dh // 2) + 2 * 2 * S * D,
        make_inputs=make_inputs, make_outputs=make_outputs, run=run,
        desc=f"Llama decoder layer bf16: S={S}, d_model={D}, {H} heads x {Dh}, SwiGLU {F}, "
             "RMSNorm, RoPE, causal attention (5 fused groups)",
        units=1, unit_name="layers",
        meta={"S": S, "D": D, "H": H, "F": F, "eps": eps})


# ------------------------------------------------------------------ counter calibration
def copy_calibration(nbytes=256 << 20) -> Workload:
    """A plain device-to-device copy of known size (torch's copy kernel): the
    reference point that scales the FETCH_SIZE / WRITE_SIZE counters to bytes."""
    n = nbytes // 4

    def make_inputs():
        return {"src": np.zeros(n, np.float32)}

    def make_outputs(d):
        import torch
        return {"dst": torch.empty(n, dtype=torch.float32, device="cuda")}

    def run(d, o, stream):
        o["dst"].copy_(d["src"])

    return Workload(name="copy_calibration_256mib", config=0, dtype="f32", flops=0,
                    bytes=2 * nbytes, make_inputs=make_inputs, make_outputs=make_outputs,
                    run=run, desc=f"device copy of {nbytes} bytes", units=1, unit_name="copies")


def all_workloads() -> list:
    """Every configuration this backend runs, in configuration order."""
    return [
        matmul_bias_relu(),
        conv3x3_bias_relu(1, "f32"), conv3x3_bias_relu(32, "f32"),
        conv3x3_bias_relu(1, "bf16"), conv3x3_bias_relu(32, "bf16"),
        irb(1), irb(32),
        qbottleneck(32),
        llama_layer(),
    ]


def holdout_workloads() -> list:
    """Shapes outside the nine configurations, each run by the same entry
    points through other launch shapes or template instances: other matmul
    aspect ratios, the conv's one-row and two-row tile kernels at other
    batches, the persistent conv at a 64-pixel and a 28-pixel row with 128
    channels, the block's other channel pairs, the int8 block at 28x28x128,
    and shorter and longer decoder layers.  The launch model's work terms are
    written from the kernels' code, not from timings of any of these."""
    import dataclasses

    def tag(w, name):
        return dataclasses.replace(w, name=name)

    return [
        matmul_bias_relu(M=512, K=1024, N=512),
        matmul_bias_relu(M=128, K=2048, N=128),
        tag(conv3x3_bias_relu(8, "f32"), "conv3x3_bias_relu_f32_n8"),
        tag(conv3x3_bias_relu(32, "f32", H=32, W=64), "conv3x3_bias_relu_f32_n32_32x64"),
        tag(conv3x3_bias_relu(16, "bf16"), "conv3x3_bias_relu_bf16_n16"),
        tag(conv3x3_bias_relu(64, "bf16", H=28, W=28, C=128, F=128),
            "conv3x3_bias_relu_bf16_n64_28x28x128"),
        tag(irb(8), "mbv2_irb_f32_n8"),
        tag(irb(16, H=28, W=28, C=32, E=192), "mbv2_irb_f32_n16_28x28x32x192"),
        tag(irb(4, H=112, W=112, C=16, E=96), "mbv2_irb_f32_n4_112x112x16x96"),
        tag(qbottleneck(8), "qbottleneck_i8_n8"),
        tag(qbottleneck(16, H=28, W=28, C=128), "qbottleneck_i8_n16_28x28x128"),
        llama_layer(S=256),
        llama_layer(S=1024),
    ]


def linalg_text(w: Workload) -> str:
    """The linalg form of a workload (npu_amd.blocks), the input of the
    reference's pipeline and cost model."""
    from . import blocks
    m = w.meta
    if w.config == 1:
        return blocks.matmul_bias_act(m["M"], m["K"], m["N"])
    if w.config == 2:
        return blocks.conv_bias_act(m["N"], m["H"], m["W"], m["C"], m["F"], elem=w.dtype)
    if w.config == 3:
        return blocks.inverted_residual(m["N"], m["H"], m["W"], m["C"], m["E"])
    if w.config == 4:
        return blocks.qbottleneck(m["N"], m["H"], m["W"], m["C"], m["M1"])
    if w.config == 5:
        return blocks.llama_layer(m["S"], m["D"], m["H"], m["F"], m["eps"])
    raise KeyError(w.name)


HEADLINE = "conv3x3_bias_relu_f32_n32"


def by_name(name: str) -> Workload:
    for w in all_workloads() + [copy_calibration()]:
        if w.name == name:
            return w
    raise KeyError(name)
