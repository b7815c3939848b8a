"""A seeded sweep of shapes for every fused-group entry point, against the
oracle with the same bounds as the hand-picked cases (fp32: rtol 1e-5 in the
error-bound form; bf16: one rounding at the output; int8: bit for bit).

The shapes are drawn once, from fixed seeds, inside what each entry point
accepts: any M, N and K a multiple of 4 (matmul); 1x1 and 3x3 filters with
and without padding, f32 channels a multiple of 4 and bf16 a multiple of 8,
any filter count, rows up to 70 pixels and batches large enough to reach the
persistent kernels (conv); the inverted residual block's three channel pairs;
the int8 bottleneck's three channel counts; Llama layers of 1-4 heads; the
plan-driven launch at the reference's own tile plans; and linalg text lowered
to npu_group_launch calls (matmul and conv, f32 and bf16).  They
cross the launch-shape boundaries the hand-picked cases sit on (row pairs
around 48 and 512, widths around 56 and 64, F around multiples of 16 and 64)
at places no one chose.
"""
import math
import random

import numpy as np
import pytest
import torch

import oracle
import refs
import npu_amd
from npu_amd import blocks, configs, groups, lower, mlir, tileplan
from npu_amd import inputs as rng
from test_gpu_parity import _dev, _host, _qb_inputs, _qb_run, _qb_wide_inputs, _widened_conv
from tolerance import RTOL_BF16, RTOL_F32, bf16, check_bf16_rounded, check_bound

pytestmark = pytest.mark.gpu

ACTS = ("none", "relu", "relu6")


def _matmul_cases(n=12, seed=2026):
    r = random.Random(seed)
    return [(r.randint(1, 300), 4 * r.randint(1, 160), r.randint(1, 300), r.choice(ACTS),
             r.random() < 0.75) for _ in range(n)]


def _conv_cases(n=16, seed=2027):
    r = random.Random(seed)
    cases = []
    while len(cases) < n:
        dtype = r.choice(("f32", "bf16"))
        step = 4 if dtype == "f32" else 8
        K = r.choice((1, 3, 3, 3))
        pad = 0 if K == 1 else r.choice((0, 1, 1))
        if r.random() < 0.35:
            # the persistent kernels' range: >= 48 row pairs, F % 64 == 0,
            # two or four 64-byte channel chunks, rows up to 64 pixels
            N, H = r.randint(4, 10), r.randint(10, 24)
            W = r.randint(20, 64)
            C = r.choice((32, 64)) if dtype == "f32" else r.choice((64, 128))
            F, K, pad = 64 * r.randint(1, 2), 3, 1
        else:
            N, H, W = r.randint(1, 6), r.randint(1, 20), r.randint(1, 70)
            C, F = step * r.randint(1, 16), r.randint(1, 130)
        if H + 2 * pad - K + 1 < 1 or W + 2 * pad - K + 1 < 1:
            continue
        cases.append((N, H, W, C, F, K, pad, r.choice(ACTS), r.random() < 0.75, dtype))
    return cases


def _irb_cases(n=6, seed=2028):
    """The tuned (C, E) pairs, then as many with any C % 4 == 0 up to 128 and
    E % 16 == 0 (the streaming kernel)."""
    r = random.Random(seed)
    tuned = [(r.randint(1, 4), r.randint(1, 20), r.randint(1, 20)) + r.choice(((24, 144), (16, 96), (32, 192)))
             for _ in range(n)]
    other = [(r.randint(1, 4), r.randint(1, 20), r.randint(1, 20), 4 * r.randint(1, 32), 16 * r.randint(1, 24))
             for _ in range(n)]
    return tuned + other


def _qb_cases(n=6, seed=2029):
    r = random.Random(seed)
    return [(r.randint(1, 3), r.randint(1, 20), r.randint(1, 20), r.choice((64, 128, 256)))
            for _ in range(n)]


def _qb_wide_cases(n=6, seed=2035):
    """(C, M1) off the tuned instances: multiples of 64 up to 640 and 256."""
    r = random.Random(seed)
    cases = []
    while len(cases) < n:
        c, m1 = 64 * r.randint(1, 10), 64 * r.randint(1, 4)
        if (c, m1) not in ((256, 64), (128, 64), (64, 64)):
            cases.append((r.randint(1, 3), r.randint(1, 16), r.randint(1, 16), c, m1))
    return cases


def _planned_cases(n=8, seed=2031):
    r = random.Random(seed)
    return [(r.randint(1, 400), r.randint(1, 1200), r.randint(1, 400)) for _ in range(n)]


def _lowered_cases(n=8, seed=2032):
    r = random.Random(seed)
    cases = []
    for _ in range(n):
        if r.random() < 0.4:
            cases.append(("matmul", r.randint(1, 200), 4 * r.randint(1, 100), r.randint(1, 200),
                          r.choice(ACTS), "f32"))
        else:
            elem = r.choice(("f32", "bf16"))
            C = (4 if elem == "f32" else 8) * r.randint(1, 12)
            cases.append(("conv", r.randint(1, 6), r.randint(1, 20), r.randint(1, 64), C,
                          r.randint(1, 100), elem))
    return cases


def _llama_cases(n=5, seed=2030):
    """Sequence lengths in 32-row blocks, then as many of any length."""
    r = random.Random(seed)
    blocks_ = [(32 * r.randint(1, 8), r.randint(1, 4), 64 * r.randint(1, 24)) for _ in range(n)]
    ragged = [(r.randint(1, 300), r.randint(1, 4), 64 * r.randint(1, 24)) for _ in range(n)]
    return blocks_ + ragged


@pytest.mark.parametrize("M,K,N,act,bias", _matmul_cases())
def test_sweep_matmul(cuda, M, K, N, act, bias):
    seed = 500 + M + K + N
    A = rng.uniform(seed, 0, (M, K), -1, 1)
    B = rng.uniform(seed, 1, (K, N), -1, 1)
    b = rng.uniform(seed, 2, (N,), -1, 1) if bias else None
    out = torch.empty(M, N, device="cuda")
    groups.fused_matmul_bias_act(_dev(A), _dev(B), None if b is None else _dev(b), out, act)
    torch.cuda.synchronize()
    ref, mag = refs.matmul_bias_act(A, B, b, act)
    check_bound(_host(out), ref, mag, RTOL_F32, what=f"matmul {M}x{K}x{N} {act}")


@pytest.mark.parametrize("N,H,W,C,F,K,pad,act,bias,dtype", _conv_cases())
def test_sweep_conv(cuda, N, H, W, C, F, K, pad, act, bias, dtype):
    seed = 600 + N * H + W + C + F
    x = rng.uniform(seed, 0, (N, H, W, C), 0, 1)
    w = rng.normal(seed, 1, (F, K, K, C), 0, math.sqrt(2 / (K * K * C)))
    b = rng.uniform(seed, 2, (F,), -0.1, 0.1) if bias else None
    if dtype == "bf16":
        x, w = rng.to_bf16_bits(x), rng.to_bf16_bits(w)
    Ho, Wo = H + 2 * pad - K + 1, W + 2 * pad - K + 1
    out = torch.empty(N, Ho, Wo, F, device="cuda",
                      dtype=torch.float32 if dtype == "f32" else torch.bfloat16)
    groups.fused_conv2d_nhwc_bias_act(_dev(x), _dev(w), None if b is None else _dev(b), out, pad,
                                      act)
    torch.cuda.synchronize()
    what = f"conv {dtype} {N}x{H}x{W}x{C}->{F} k{K} p{pad} {act}"
    ref, mag = refs.conv_bias_act(x, w, b, pad, act)
    if dtype == "f32":
        check_bound(_host(out), ref, mag, RTOL_F32, what=what)
    else:
        ref32, _ = _widened_conv(x, w, b, pad, act)
        check_bf16_rounded(_host(out), ref32, mag, K * K * C + 1, what=what)


@pytest.mark.parametrize("N,H,W,C,E", _irb_cases())
def test_sweep_irb(cuda, N, H, W, C, E):
    seed = 700 + N * H + W + C
    x = rng.uniform(seed, 0, (N, H, W, C), 0, 1)
    we = rng.normal(seed, 1, (E, C), 0, math.sqrt(2 / C))
    wdw = rng.normal(seed, 2, (3, 3, E), 0, math.sqrt(2 / 9))
    wp = rng.normal(seed, 3, (C, E), 0, math.sqrt(2 / E))
    d = configs.to_device({"x": x, "we": we, "wdw": wdw, "wp": wp})
    out = torch.empty_like(d["x"])
    groups.fused_irb_f32(d["x"], d["we"], d["wdw"], d["wp"], out)
    torch.cuda.synchronize()
    ref, mag = refs.irb(x, we, wdw, wp)
    check_bound(_host(out), ref, mag, RTOL_F32, what=f"irb {N}x{H}x{W}x{C}/{E}")


@pytest.mark.parametrize("N,H,W,C", _qb_cases())
def test_sweep_int8_bottleneck(cuda, N, H, W, C):
    inp = _qb_inputs(N, H, W, C, 64, 800 + N * H + W + C)
    ref = oracle.block_qbottleneck(**inp)
    assert np.array_equal(_qb_run(inp), ref), f"int8 bottleneck {N}x{H}x{W}x{C}"


@pytest.mark.parametrize("N,H,W,C,M1", _qb_wide_cases())
def test_sweep_int8_bottleneck_wide(cuda, N, H, W, C, M1):
    inp = _qb_wide_inputs(N, H, W, C, M1, 850 + N * H + W + C + M1)
    ref = oracle.block_qbottleneck(**inp)
    assert np.array_equal(_qb_run(inp), ref), f"int8 bottleneck {N}x{H}x{W}x{C}/{M1}"


@pytest.mark.parametrize("S,H,F", _llama_cases())
def test_sweep_llama_layer(cuda, S, H, F):
    D = 64 * H
    w = configs.llama_layer(S=S, D=D, H=H, F=F, seed=900 + S + F)
    inp = w.make_inputs()
    d = configs.to_device(inp)
    o = w.make_outputs(d)
    groups.llama_layer(d, o, H, 1e-5)
    torch.cuda.synchronize()
    for name, (ref, mag) in refs.llama_reference(inp, H, 1e-5).items():
        check_bound(bf16(_host(o[name])), bf16(ref), mag, RTOL_BF16, what=f"layer S{S} H{H} F{F} {name}")


@pytest.mark.parametrize("M,K,N", _planned_cases())
def test_sweep_planned_matmul(cuda, M, K, N):
    """The group through the reference's own plan for its shape: within the
    f32 bound of the oracle, or refused by name before any launch (a plan
    that spills to DRAM, or a tile of more 16x16 blocks than the launch
    holds)."""
    try:
        p = tileplan.matmul_group_plan(mlir.parse_functions(blocks.matmul_bias_act(M, K, N))[0])
    except NotImplementedError as e:
        assert "spills" in str(e), e
        return
    seed = 1000 + M + K + N
    A = rng.uniform(seed, 0, (M, K), -1, 1)
    B = rng.uniform(seed, 1, (K, N), -1, 1)
    b = rng.uniform(seed, 2, (N,), -1, 1)
    out = torch.empty((M, N), dtype=torch.float32, device="cuda")
    try:
        groups.planned_matmul_bias_act(_dev(A), _dev(B), _dev(b), out, p["plan"], "relu")
    except npu_amd.NpuError as e:
        assert "blocks" in str(e), e
        return
    torch.cuda.synchronize()
    ref, mag = refs.matmul_bias_act(A, B, b, "relu")
    check_bound(_host(out), ref, mag, RTOL_F32, what=f"planned matmul {M}x{K}x{N} tile {p['tile']}")


@pytest.mark.parametrize("case", _lowered_cases())
def test_sweep_lowered(cuda, case):
    """linalg text -> npu_amd.lower -> npu_group_launch, against the oracle."""
    kind = case[0]
    if kind == "matmul":
        _, M, K, N, act, _ = case
        seed = 1100 + M + K + N
        A = rng.uniform(seed, 0, (M, K), -1, 1)
        B = rng.uniform(seed, 1, (K, N), -1, 1)
        b = rng.uniform(seed, 2, (N,), -1, 1)
        prog = lower.lower_text(blocks.matmul_bias_act(M, K, N, act=act))
        out = prog.run({"A": _dev(A), "B": _dev(B), "bias": _dev(b)})["%y"]
        torch.cuda.synchronize()
        ref, mag = refs.matmul_bias_act(A, B, b, act)
        check_bound(_host(out), ref, mag, RTOL_F32, what=f"lowered matmul {M}x{K}x{N}")
        return
    _, N, H, W, C, F, elem = case
    seed = 1200 + N * H + W + C + F
    x = rng.uniform(seed, 0, (N, H, W, C), 0, 1)
    w = rng.normal(seed, 1, (F, 3, 3, C), 0, math.sqrt(2 / (9 * C)))
    b = rng.uniform(seed, 2, (F,), -0.1, 0.1)
    if elem == "bf16":
        x, w, b = rng.to_bf16_bits(x), rng.to_bf16_bits(w), rng.to_bf16_bits(b)
    prog = lower.lower_text(blocks.conv_bias_act(N, H, W, C, F, elem=elem))
    out = prog.run({"x": _dev(x), "w": _dev(w), "bias": _dev(b)})["%y"]
    torch.cuda.synchronize()
    bias32 = bf16(b).astype(np.float32) if elem == "bf16" else b
    ref, mag = refs.conv_bias_act(x, w, bias32, 1, "relu")
    what = f"lowered conv {elem} {N}x{H}x{W}x{C}->{F}"
    if elem == "f32":
        check_bound(_host(out), ref, mag, RTOL_F32, what=what)
    else:
        ref32, _ = _widened_conv(x, w, bias32, 1, "relu")
        check_bf16_rounded(_host(out), ref32, mag, 9 * C + 1, what=what)
