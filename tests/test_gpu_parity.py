"""GPU parity of the fused-group kernels against the CPU restatement.

Every call goes through the C-ABI (npu_amd.groups -> libnpu_amd.so).  fp32
results must lie within rtol 1e-5 and bf16 within rtol 2e-2 of the oracle in
the error-bound form of tests/tolerance.py; integer results bit for bit.
Configuration sizes run in full; batch-32 runs check every image against
the oracle's OpenMP build (bit-identical to the single-thread one), plus
size-independent properties.
"""
import math

import numpy as np
import pytest
import torch

import oracle
import refs
from npu_amd import blocks, configs, frontend, groups, lower, mlir
from npu_amd import inputs as rng
from tolerance import RTOL_BF16, RTOL_F32, bf16, check_bf16_rounded, check_bf16_stage, check_bound

pytestmark = pytest.mark.gpu


def _dev(a):
    return configs.to_device({"a": a})["a"]


def _host(t):
    return configs.to_host(t)


def _widened_conv(x_bits, w_bits, b, pad, act):
    """The oracle's f32 value of a bf16 conv chain before its final rounding:
    the f32 loops over the inputs widened to f32 (bf16 x bf16 products are
    exact in f32, summed in the same order)."""
    return refs.conv_bias_act(bf16(x_bits).astype(np.float32), bf16(w_bits).astype(np.float32),
                              b, pad, act)


def _run_workload(w):
    arrs = w.make_inputs()
    d = configs.to_device(arrs)
    o = w.make_outputs(d)
    w.run(d, o, None)
    torch.cuda.synchronize()
    return arrs, {k: _host(v) for k, v in o.items()}


# ------------------------------------------------------------------ C1
def test_c1_matmul_bias_relu_config(cuda):
    w = configs.matmul_bias_relu()
    arrs, out = _run_workload(w)
    ref, mag = refs.reference(w.name, arrs)["out"]
    check_bound(out["out"], ref, mag, RTOL_F32, what=w.name)
    assert (out["out"] == 0).any() and (out["out"] > 0).any()


@pytest.mark.parametrize("M,K,N,act,bias", [
    (37, 20, 45, "relu", True),      # ragged M, N and a K that is not a multiple of 16
    (16, 4, 16, "none", False),      # smallest K, no bias
    (64, 4096, 32, "relu6", True),   # long K, ReLU6
    (1, 512, 256, "relu", True),     # single row
    (20, 400, 36, "relu", True),     # K in whole chunks, a wave's last batch partial
    (5, 64, 4, "none", True),        # N = 4: the narrowest 16-byte B rows
    (33, 48, 3, "relu", False),      # N < 4: B read a value at a time
])
def test_c1_matmul_shapes(cuda, M, K, N, act, bias):
    A = rng.uniform(11, 0, (M, K), -1, 1)
    B = rng.uniform(11, 1, (K, N), -1, 1)
    b = rng.uniform(11, 2, (N,), -1, 1) if bias else None
    out = torch.empty(M, N, device="cuda")
    groups.fused_matmul_bias_act(_dev(A), _dev(B), None if b is None else _dev(b), out, act)
    torch.cuda.synchronize()
    ref, mag = refs.matmul_bias_act(A, B, b, act)
    check_bound(_host(out), ref, mag, RTOL_F32, what=f"matmul {M}x{K}x{N}")


def test_c1_reference_kat_fills(cuda):
    """e2e_verify's closed form on the GPU: fills 0.01 / 0.02 give K * 2e-4."""
    M, K, N = 256, 512, 256
    A = torch.full((M, K), 0.01, device="cuda")
    B = torch.full((K, N), 0.02, device="cuda")
    out = torch.empty(M, N, device="cuda")
    groups.fused_matmul_bias_act(A, B, None, out, "relu")
    np.testing.assert_allclose(_host(out), K * 0.01 * 0.02, atol=1e-4, rtol=1e-3)


# ------------------------------------------------------------------ C2
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_c2_conv_config_n1(cuda, dtype):
    w = configs.conv3x3_bias_relu(1, dtype)
    arrs, out = _run_workload(w)
    ref, mag = refs.reference(w.name, arrs)["out"]
    if dtype == "f32":
        check_bound(out["out"], ref, mag, RTOL_F32, what=w.name)
    else:
        ref32, _ = _widened_conv(arrs["x"], arrs["w"], arrs["bias"], 1, "relu")
        check_bf16_rounded(out["out"], ref32, mag, 9 * 64 + 1, what=w.name)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_c2_conv_config_n32(cuda, dtype):
    w = configs.conv3x3_bias_relu(32, dtype)
    arrs, out = _run_workload(w)
    with oracle.threaded():
        ref, mag = refs.reference(w.name, arrs)["out"]
        got = out["out"]
        if dtype == "f32":
            check_bound(got, ref, mag, RTOL_F32, what=w.name)
        else:
            ref32, _ = _widened_conv(arrs["x"], arrs["w"], arrs["bias"], 1, "relu")
            check_bf16_rounded(got, ref32, mag, 9 * 64 + 1, what=w.name)
    # size-independent property over the whole batch: ReLU output, finite,
    # and image i's result depends only on image i (batch permutation commutes)
    full = out["out"] if dtype == "f32" else bf16(out["out"])
    assert np.isfinite(full).all() and (full >= 0).all()
    x = configs.to_device(arrs)
    perm = torch.arange(31, -1, -1, device="cuda")
    xp = x["x"][perm].contiguous()
    o2 = torch.empty_like(w.make_outputs(x)["out"])
    groups.fused_conv2d_nhwc_bias_act(xp, x["w"], x["bias"], o2, 1, "relu")
    torch.cuda.synchronize()
    assert np.array_equal(_host(o2), out["out"][::-1])


@pytest.mark.parametrize("N,H,W,C,F,K,pad,act,bias,dtype", [
    (2, 5, 7, 16, 16, 3, 1, "relu", True, "f32"),    # tiny, non-square, one F block
    (1, 9, 6, 32, 48, 3, 1, "relu6", True, "f32"),   # F not a multiple of 64
    (3, 8, 8, 16, 32, 1, 0, "none", False, "f32"),   # 1x1, no pad, no bias
    (1, 6, 6, 16, 16, 3, 0, "relu", True, "f32"),    # valid (unpadded) conv
    (2, 5, 7, 32, 16, 3, 1, "relu", True, "bf16"),
    (1, 9, 6, 64, 80, 3, 1, "relu6", False, "bf16"),
    # 3x3/pad-1 LDS-halo kernel: the 2-row x 64-filter shape needs >= 512 row
    # pairs; an odd H leaves a half tile at the bottom of each image
    (64, 17, 9, 16, 64, 3, 1, "relu", True, "f32"),
    (64, 17, 9, 32, 80, 3, 1, "relu", True, "bf16"),
    # the persistent kernel (>= 48 row pairs, F a multiple of 64, C two or
    # four 64-byte chunks) at a run-time width, an odd H, two 64-filter
    # blocks, a 64-wide row and four bf16 chunks; and with fewer rows than
    # workgroups (ranges of zero or one row)
    (64, 17, 9, 32, 128, 3, 1, "relu", True, "f32"),
    (2, 56, 56, 64, 64, 3, 1, "relu", True, "f32"),
    (3, 33, 56, 32, 64, 3, 1, "relu", True, "f32"),
    (2, 56, 56, 64, 64, 3, 1, "relu", True, "bf16"),
    (4, 28, 28, 128, 128, 3, 1, "relu", True, "bf16"),
    (64, 17, 30, 64, 64, 3, 1, "relu", True, "f32"),  # 64 channels at a run-time width
    (32, 32, 64, 64, 64, 3, 1, "relu", True, "f32"),
    (40, 26, 60, 64, 64, 3, 1, "relu6", False, "bf16"),
    (64, 16, 20, 128, 64, 3, 1, "none", True, "bf16"),
    (1, 3, 64, 16, 32, 3, 1, "relu", True, "f32"),    # widest row the LDS tile holds
    (1, 4, 70, 16, 16, 3, 1, "relu", True, "f32"),    # wider: general kernel
    (2, 6, 66, 32, 16, 3, 1, "relu", True, "bf16"),
])
def test_c2_conv_shapes(cuda, N, H, W, C, F, K, pad, act, bias, dtype):
    x = rng.uniform(12, 0, (N, H, W, C), 0, 1)
    w = rng.normal(12, 1, (F, K, K, C), 0, math.sqrt(2 / (K * K * C)))
    b = rng.uniform(12, 2, (F,), -0.1, 0.1) if bias else None
    if dtype == "bf16":
        x, w = rng.to_bf16_bits(x), rng.to_bf16_bits(w)
    Ho, Wo = H + 2 * pad - K + 1, W + 2 * pad - K + 1
    out = torch.empty(N, Ho, Wo, F, device="cuda",
                      dtype=torch.float32 if dtype == "f32" else torch.bfloat16)
    groups.fused_conv2d_nhwc_bias_act(_dev(x), _dev(w), None if b is None else _dev(b), out, pad,
                                      act)
    torch.cuda.synchronize()
    ref, mag = refs.conv_bias_act(x, w, b, pad, act)
    if dtype == "f32":
        check_bound(_host(out), ref, mag, RTOL_F32, what="conv")
    else:
        ref32, _ = _widened_conv(x, w, b, pad, act)
        check_bf16_rounded(_host(out), ref32, mag, K * K * C + 1, what="conv")


@pytest.mark.parametrize("N,H,W,C,F", [(2, 5, 7, 16, 16), (64, 17, 9, 32, 128)])
def test_c2_nan_propagates(cuda, N, H, W, C, F):
    """arith.maximumf propagates NaN: a NaN input pixel makes every output
    of its 3x3 neighbourhood NaN through the ReLU, in the oracle and here
    (rows kernel and persistent kernel)."""
    x = rng.uniform(13, 0, (N, H, W, C), 0, 1)
    x[N - 1, H // 2, W // 2, C - 1] = np.nan
    w = rng.normal(13, 1, (F, 3, 3, C), 0, math.sqrt(2 / (9 * C)))
    b = rng.uniform(13, 2, (F,), -0.1, 0.1)
    out = torch.empty(N, H, W, F, device="cuda", dtype=torch.float32)
    groups.fused_conv2d_nhwc_bias_act(_dev(x), _dev(w), _dev(b), out, 1, "relu")
    torch.cuda.synchronize()
    got = _host(out)
    ref, mag = refs.conv_bias_act(x, w, b, 1, "relu")
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.isnan(ref).sum() == 9 * F
    ok = ~np.isnan(ref)
    check_bound(got[ok], ref[ok], mag[ok], RTOL_F32, what="conv with NaN")


def _same_f32(a, b):
    """Bit-identical f32 arrays, any NaN equal to any NaN (the oracle's
    maximumf returns the canonical NaN)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a)
    return np.array_equal(nan, np.isnan(b)) and np.array_equal(a.view(np.uint32)[~nan],
                                                               b.view(np.uint32)[~nan])


@pytest.mark.parametrize("kind", ["full_mantissa", "wide_exponents", "constant",
                                  "near_subnormal_x", "near_subnormal_w", "tiny_products",
                                  "subnormal_bias"])
def test_c2_f32_bf16_split_parity(cuda, kind):
    """The f32 persistent conv multiplies on the bf16 pipe with each value
    split into three bf16 parts (six part products), within the f32 bound:
    values whose 24-bit significands are all used, values spread over
    2^-20..2^20 and constant inputs (every product rounds the same way, so
    dropped terms add up coherently).  Values outside the split's domain
    (zero, or magnitudes in [2^-55, 2^55)) are carried by the kernel's
    exact path, bit-identical to the oracle: inputs of 2^-118 times
    filters of 2^100, filters of 2^-118 (with f32 subnormals among them)
    times inputs of 2^100, inputs and filters of 2^-60 (products near
    f32's subnormals), and a subnormal bias."""
    N, H, W, C, F = 64, 16, 56, 64, 64
    x = rng.uniform(15, 0, (N, H, W, C), 0.5, 1)
    w = rng.normal(15, 1, (F, 3, 3, C), 0, math.sqrt(2 / (9 * C)))
    b = rng.uniform(15, 2, (F,), -0.1, 0.1)
    exact = True
    if kind == "full_mantissa":
        # set every low significand bit: the h and m parts both matter
        x = (x.view(np.uint32) | np.uint32(0x7FFF)).view(np.float32)
        w = (w.view(np.uint32) | np.uint32(0x7FFF)).view(np.float32)
        exact = False
    elif kind == "wide_exponents":
        e = rng.randint(15, 3, (N, H, W, C), -20, 20)
        x = (x * np.exp2(e)).astype(np.float32)
        exact = False
    elif kind.startswith("near_subnormal"):
        tiny, big = np.float32(2.0 ** -118), np.float32(2.0 ** 100)
        x = (x.view(np.uint32) | np.uint32(0x7FFF)).view(np.float32)
        w = (w.view(np.uint32) | np.uint32(0x7FFF)).view(np.float32)
        if kind == "near_subnormal_x":
            x, w = (x * tiny).astype(np.float32), (w * big).astype(np.float32)
        else:
            x, w = (x * big).astype(np.float32), (w * tiny).astype(np.float32)
        b = (b * np.float32(2.0 ** -18)).astype(np.float32)
    elif kind == "tiny_products":
        x = (x * np.float32(2.0 ** -60)).astype(np.float32)
        w = (w * np.float32(2.0 ** -60)).astype(np.float32)
        b = np.zeros_like(b)
    elif kind == "subnormal_bias":
        b = (b * np.float32(2.0 ** -130)).astype(np.float32)
        x[:] = 0
    else:
        x = np.full((N, H, W, C), 1.0 + 2.0 ** -9 + 2.0 ** -17 + 2.0 ** -23, np.float32)
        w = np.full((F, 3, 3, C), -(0.75 + 2.0 ** -10 + 2.0 ** -19 + 2.0 ** -22) / 64, np.float32)
        exact = False
    out = torch.empty(N, H, W, F, device="cuda", dtype=torch.float32)
    groups.fused_conv2d_nhwc_bias_act(_dev(x), _dev(w), _dev(b), out, 1, "none")
    torch.cuda.synchronize()
    got = _host(out)
    with oracle.threaded():
        ref, mag = refs.conv_bias_act(x, w, b, 1, "none")
    check_bound(got, ref, mag, RTOL_F32, what=f"f32 conv, {kind}")
    if exact:
        assert _same_f32(got, ref), f"f32 conv, {kind}: exact path not bit-identical to the oracle"


@pytest.mark.parametrize("case", ["inf_x", "neg_inf_x", "inf_times_zero", "inf_w", "nan_w",
                                  "inf_bias", "mixed_inf"])
def test_c2_f32_non_finite_values(cuda, case):
    """Inf and NaN in the f32 persistent conv follow the f32 loops: an
    infinite input gives +-Inf in every output it reaches (NaN where it
    meets a zero filter value or an opposite infinity, as Inf * 0 and
    Inf - Inf do in the oracle), an infinite or NaN filter value or bias
    likewise.  Outputs next to such a value come from the kernel's exact
    path and equal the oracle's bit for bit (NaN as NaN); the rest stay
    within the f32 bound."""
    N, H, W, C, F = 64, 16, 56, 64, 64
    x = rng.uniform(16, 0, (N, H, W, C), 0, 1)
    w = rng.normal(16, 1, (F, 3, 3, C), 0, math.sqrt(2 / (9 * C)))
    b = rng.uniform(16, 2, (F,), -0.1, 0.1)
    if case == "inf_x":
        x[3, 7, 20, 5] = np.inf
    elif case == "neg_inf_x":
        x[3, 0, 55, 63] = -np.inf       # a corner: only four taps reach it
    elif case == "inf_times_zero":
        x[3, 7, 20, 5] = np.inf
        w[:8, 1, 1, 5] = 0.0            # filters 0..7 meet it with a zero at the centre tap
    elif case == "inf_w":
        w[17, 2, 0, 9] = np.inf
    elif case == "nan_w":
        w[40, 0, 2, 33] = np.nan
    elif case == "inf_bias":
        b[5] = -np.inf
    elif case == "mixed_inf":
        x[3, 7, 20, 5] = np.inf
        x[3, 8, 20, 5] = -np.inf        # filters meet both: +Inf - Inf = NaN where both signs agree
    out = torch.empty(N, H, W, F, device="cuda", dtype=torch.float32)
    groups.fused_conv2d_nhwc_bias_act(_dev(x), _dev(w), _dev(b), out, 1, "none")
    torch.cuda.synchronize()
    got = _host(out)
    with oracle.threaded():
        ref, mag = refs.conv_bias_act(x, w, b, 1, "none")
    hit = ~np.isfinite(ref)
    assert hit.any()
    assert np.array_equal(np.isnan(got), np.isnan(ref)), f"{case}: NaN positions differ"
    assert np.array_equal(got[hit & ~np.isnan(ref)], ref[hit & ~np.isnan(ref)]), f"{case}: Inf values differ"
    ok = ~hit
    check_bound(got[ok], ref[ok], mag[ok], RTOL_F32, what=f"f32 conv next to {case}")
    # the rows the exact path ran (every row of a launch whose filters or bias
    # hold a non-finite value) are bit-identical
    if case in ("inf_w", "nan_w"):
        assert _same_f32(got, ref)


def test_c1_nan_propagates(cuda):
    A = rng.uniform(14, 0, (64, 128), -1, 1)
    A[5, 17] = np.nan
    B = rng.uniform(14, 1, (128, 64), -1, 1)
    out = torch.empty(64, 64, device="cuda", dtype=torch.float32)
    groups.fused_matmul_bias_act(_dev(A), _dev(B), None, out, "relu")
    torch.cuda.synchronize()
    got = _host(out)
    assert np.isnan(got[5]).all() and not np.isnan(np.delete(got, 5, axis=0)).any()


def test_c2_reference_kat_fills(cuda):
    """numerical_verify's conv closed form (fills 0.01/0.02, unpadded) at C=16:
    every output is C*KH*KW*0.01*0.02."""
    x = torch.full((1, 6, 6, 16), 0.01, device="cuda")
    w = torch.full((16, 3, 3, 16), 0.02, device="cuda")
    out = torch.empty(1, 4, 4, 16, device="cuda")
    groups.fused_conv2d_nhwc_bias_act(x, w, None, out, 0, "none")
    np.testing.assert_allclose(_host(out), 16 * 9 * 0.01 * 0.02, atol=1e-5)


# ------------------------------------------------------------------ C4
def _qb_inputs(N, H, W, C, M1, seed):
    x = rng.randint(seed, 0, (N, H, W, C), 0, 127).astype(np.int8)
    w1 = rng.randint(seed, 1, (M1, C), -127, 127).astype(np.int8)
    w2 = rng.randint(seed, 2, (M1, 3, 3, M1), -127, 127).astype(np.int8)
    w3 = rng.randint(seed, 3, (C, M1), -127, 127).astype(np.int8)
    q = {}
    for i, (k, n, sh) in enumerate((("1", M1, 24), ("2", M1, 26), ("3", C, 26))):
        q["m" + k] = rng.randint(seed, 4 + i, (n,), 2 ** 30, 2 ** 31 - 1).astype(np.int32)
        q["s" + k] = rng.randint(seed, 7 + i, (n,), sh, sh + 3).astype(np.int32)
    return dict(x=x, w1=w1, w2=w2, w3=w3, **q)


def _qb_run(inp):
    d = configs.to_device(inp)
    out = torch.empty_like(d["x"])
    groups.fused_qbottleneck_i8(d["x"], d["w1"], d["w2"], d["w3"], d["m1"], d["s1"], d["m2"],
                                d["s2"], d["m3"], d["s3"], out)
    torch.cuda.synchronize()
    return _host(out)


def test_c4_qbottleneck_config_n32(cuda):
    w = configs.qbottleneck(32)
    arrs, out = _run_workload(w)
    with oracle.threaded():
        ref = refs.qbottleneck(arrs)
    assert np.array_equal(out["out"], ref), "int8 bottleneck must be bit-exact"
    # whole batch: output range and batch-permutation commutation (bit-exact)
    assert out["out"].min() >= 0
    d = configs.to_device(arrs)
    perm = torch.arange(31, -1, -1, device="cuda")
    inp2 = dict(arrs, x=_host(d["x"][perm].contiguous()))
    assert np.array_equal(_qb_run(inp2), out["out"][::-1])


@pytest.mark.parametrize("N,H,W,C,M1", [
    (2, 9, 13, 256, 64),   # ragged tiles on both spatial dims
    (1, 8, 8, 64, 64),     # exactly one tile
    (3, 5, 3, 128, 64),    # image smaller than a tile
    (1, 1, 1, 256, 64),    # single pixel: only the centre tap sees data
])
def test_c4_qbottleneck_shapes(cuda, N, H, W, C, M1):
    inp = _qb_inputs(N, H, W, C, M1, 21 + H)
    ref = oracle.block_qbottleneck(**inp)
    assert np.array_equal(_qb_run(inp), ref)


def test_c4_requant_extremes(cuda):
    """Shifts at both ends of the TOSA range and multipliers at the int32
    limits: the kernel's 64-bit rounding must match the oracle bit for bit."""
    N, H, W, C, M1 = 1, 8, 8, 256, 64
    inp = _qb_inputs(N, H, W, C, M1, 77)
    inp["m1"][:] = 2 ** 31 - 1
    inp["s1"][:] = rng.randint(78, 0, (M1,), 36, 62).astype(np.int32)
    inp["m2"][:8] = 0
    inp["s2"][:] = 30
    # low end of the shift range with multipliers small enough that the
    # rescaled value still fits int32 (the apply_scale precondition)
    inp["m3"][:] = rng.randint(79, 0, (C,), 1, 4096).astype(np.int32)
    inp["s3"][:] = 2
    ref = oracle.block_qbottleneck(**inp)
    assert np.array_equal(_qb_run(inp), ref)


def test_c4_requant_wide_products(cuda):
    """Shifts from 33 to 62 with multipliers at the int32 limits of either
    sign and zero, and accumulators at their extremes (x and the filters at
    +-127): products that need all 64 bits, bit for bit against the
    oracle's rounding."""
    N, H, W, C, M1 = 1, 8, 8, 256, 64
    inp = _qb_inputs(N, H, W, C, M1, 81)
    inp["x"][:] = 127
    inp["w1"][::2] = 127
    inp["w1"][1::2] = -127
    inp["m1"][:] = rng.randint(82, 0, (M1,), 1 << 24, 1 << 30).astype(np.int32)
    inp["m1"][:4] = [2 ** 31 - 1, -(2 ** 31), 0, 1]
    inp["s1"][:] = rng.randint(83, 0, (M1,), 33, 63).astype(np.int32)
    inp["s1"][:4] = [33, 62, 33, 62]
    inp["m2"][:] = 2 ** 31 - 1
    inp["s2"][:] = 33
    inp["m3"][:] = -(2 ** 30)
    inp["s3"][:] = rng.randint(84, 0, (C,), 33, 40).astype(np.int32)
    ref = oracle.block_qbottleneck(**inp)
    assert np.array_equal(_qb_run(inp), ref)


def _qb_wide_inputs(N, H, W, C, M1, seed):
    """Inputs for wide channel counts: each stage's shift set from its
    reduction length K so that requantized values land mid-range (an
    accumulator's spread grows as sqrt(K)), not all clamped."""
    inp = _qb_inputs(N, H, W, C, M1, seed)
    for i, (k, n, K) in enumerate((("1", M1, C), ("2", M1, 9 * M1), ("3", C, M1))):
        base = int(round(24.5 + math.log2(5329.0 * math.sqrt(K))))
        inp["s" + k] = rng.randint(seed, 20 + i, (n,), base - 1, base + 1).astype(np.int32)
    return inp


@pytest.mark.parametrize("N,H,W,C,M1", [
    (1, 9, 10, 512, 128),    # ResNet-50's later bottlenecks
    (1, 7, 7, 1024, 256),
    (1, 7, 7, 2048, 512),
    (2, 6, 13, 192, 64),     # C off the tuned instances
    (3, 11, 5, 128, 128),
    (8, 20, 20, 64, 192),    # more tiles than resident workgroups
])
def test_c4_qbottleneck_any_channels(cuda, N, H, W, C, M1):
    """(C, M1) outside the tuned instances run on the kernel that reads its
    filter blocks from L2 where they are used: bit for bit against the
    oracle, with most requantized values off the clamp bounds."""
    inp = _qb_wide_inputs(N, H, W, C, M1, 90 + C // 64)
    print(f"qbottleneck stream {N}x{H}x{W}x{C}/{M1}", flush=True)
    ref = oracle.block_qbottleneck(**inp)
    got = _qb_run(inp)
    assert np.array_equal(got, ref)
    inner = ((ref > 0) & (ref < 127)).mean()
    assert inner > 0.2, f"only {inner:.0%} of the outputs off the clamp bounds"


# ------------------------------------------------------------------ C3
def test_c3_irb_config_n1(cuda):
    w = configs.irb(1)
    arrs, out = _run_workload(w)
    ref, mag = refs.reference(w.name, arrs)["out"]
    check_bound(out["out"], ref, mag, RTOL_F32, what=w.name)


def test_c3_irb_config_n32(cuda):
    w = configs.irb(32)
    arrs, out = _run_workload(w)
    with oracle.threaded():
        ref, mag = refs.reference(w.name, arrs)["out"]
    check_bound(out["out"], ref, mag, RTOL_F32, what=w.name)
    assert np.isfinite(out["out"]).all()


@pytest.mark.parametrize("N,H,W,C,E", [
    (2, 9, 13, 24, 144),   # ragged tiles (4 x 4 tiles: fewer 8 x 8 tiles than CUs)
    (1, 3, 5, 24, 144),    # image smaller than a tile
    (4, 33, 30, 24, 144),  # 4 x 4 tiles, more of them than CUs (a walk of one or two per workgroup)
    (2, 56, 56, 16, 96),
    (2, 8, 8, 16, 96),     # other block widths of the network
    (1, 10, 7, 32, 192),
    (16, 30, 30, 24, 144),  # 8 x 8 tiles (256 of them), ragged at the image edge
    (8, 44, 50, 16, 96),
    (20, 31, 30, 32, 192),
])
def test_c3_irb_shapes(cuda, N, H, W, C, E):
    x = rng.uniform(31, 0, (N, H, W, C), 0, 1)
    we = rng.normal(31, 1, (E, C), 0, math.sqrt(2 / C))
    wdw = rng.normal(31, 2, (3, 3, E), 0, math.sqrt(2 / 9))
    wp = rng.normal(31, 3, (C, E), 0, math.sqrt(2 / E))
    d = configs.to_device({"x": x, "we": we, "wdw": wdw, "wp": wp})
    out = torch.empty_like(d["x"])
    groups.fused_irb_f32(d["x"], d["we"], d["wdw"], d["wp"], out)
    torch.cuda.synchronize()
    ref, mag = refs.irb(x, we, wdw, wp)
    check_bound(_host(out), ref, mag, RTOL_F32, what=f"irb {N}x{H}x{W}x{C}/{E}")


@pytest.mark.parametrize("N,H,W,C,E", [
    (2, 9, 13, 64, 384),    # the MobileNetV2 blocks the tuned instances do not cover
    (1, 14, 14, 96, 576),
    (1, 7, 7, 160, 960),
    (3, 10, 11, 40, 240),
    (1, 12, 12, 28, 64),    # C off the 16-channel blocks
    (2, 5, 6, 8, 16),       # fewer chunks than waves
    (1, 6, 5, 320, 1280),   # the largest C
    (4, 30, 31, 24, 96),    # more tiles than resident workgroups
])
def test_c3_irb_any_channels(cuda, N, H, W, C, E):
    """(C, E) outside the tuned instances run on the kernel that streams the
    expanded channels in chunks of 16: within the f32 bound of the oracle."""
    x = rng.uniform(33, 0, (N, H, W, C), -1, 1)
    we = rng.normal(33, 1, (E, C), 0, math.sqrt(2 / C))
    wdw = rng.normal(33, 2, (3, 3, E), 0, math.sqrt(2 / 9))
    wp = rng.normal(33, 3, (C, E), 0, math.sqrt(2 / E))
    d = configs.to_device({"x": x, "we": we, "wdw": wdw, "wp": wp})
    out = torch.empty_like(d["x"])
    print(f"irb stream {N}x{H}x{W}x{C}/{E}", flush=True)
    groups.fused_irb_f32(d["x"], d["we"], d["wdw"], d["wp"], out)
    torch.cuda.synchronize()
    ref, mag = refs.irb(x, we, wdw, wp)
    check_bound(_host(out), ref, mag, RTOL_F32, what=f"irb {N}x{H}x{W}x{C}/{E}")


def test_c3_irb_relu6_clamps_both_sides(cuda):
    """Large weights drive the expand and depthwise stages past 6 and below 0."""
    N, H, W, C, E = 1, 8, 8, 24, 144
    x = rng.uniform(32, 0, (N, H, W, C), 0, 4)
    we = rng.normal(32, 1, (E, C), 0, 2.0)
    wdw = rng.normal(32, 2, (3, 3, E), 0, 2.0)
    wp = rng.normal(32, 3, (C, E), 0, 0.1)
    d = configs.to_device({"x": x, "we": we, "wdw": wdw, "wp": wp})
    out = torch.empty_like(d["x"])
    groups.fused_irb_f32(d["x"], d["we"], d["wdw"], d["wp"], out)
    torch.cuda.synchronize()
    ref, mag = refs.irb(x, we, wdw, wp)
    check_bound(_host(out), ref, mag, RTOL_F32, what="irb clamps")


# ------------------------------------------------------------------ C5
LL_H, LL_EPS = 8, 1e-5


@pytest.fixture(scope="module")
def llama_case():
    w = configs.llama_layer()
    inp = w.make_inputs()
    st = refs.llama_stages(inp, LL_H, LL_EPS)
    st["exact"] = refs.llama_stage_exact(inp, st, LL_H, LL_EPS)
    return w, inp, st


def _bf_dev(shape):
    return torch.empty(shape, dtype=torch.bfloat16, device="cuda")


def test_c5_stage_qkv_rope(cuda, llama_case):
    w, inp, st = llama_case
    d = configs.to_device(inp)
    S, D = inp["x"].shape
    Q, K, V = _bf_dev((S, D)), _bf_dev((S, D)), _bf_dev((S, D))
    groups.fused_llama_qkv_rope(d["x"], d["g1"], d["wq"], d["wk"], d["wv"], d["cos_t"],
                                d["sin_t"], Q, K, V, LL_EPS)
    torch.cuda.synchronize()
    xn = refs.normed_bf16(inp["x"], inp["g1"], LL_EPS)
    for name, t, wname, rope in (("Q", Q, "wq", True), ("K", K, "wk", True), ("V", V, "wv", False)):
        mag = refs.mag_qkv(xn, inp[wname], inp["cos_t"], inp["sin_t"], rope)
        check_bf16_stage(_host(t), st["exact"][name], mag, D + 2, what=name)
    # position 0 is not rotated: Q row 0 equals the plain projection's rounding
    q0 = bf16(_host(Q))[0]
    plain0 = bf16(xn)[0] @ bf16(inp["wq"])
    assert np.allclose(q0, plain0, rtol=1e-2, atol=1e-3)


def test_c5_stage_attention(cuda, llama_case):
    w, inp, st = llama_case
    d = configs.to_device({k: st[k] for k in ("Q", "K", "V")})
    A = _bf_dev(st["A"].shape)
    groups.fused_llama_attention(d["Q"], d["K"], d["V"], A, LL_H, 0.125)
    torch.cuda.synchronize()
    mag = refs.mag_attention(st["Q"], st["K"], st["V"], LL_H)
    S, D = st["A"].shape
    check_bf16_stage(_host(A), st["exact"]["A"], mag, S + D // LL_H, what="attention")
    # causal: row 0 attends only to key 0, so it equals V's row 0 exactly
    assert np.array_equal(_host(A)[0], st["V"][0])


@pytest.mark.parametrize("S,D,H", [(256, 512, 4), (100, 256, 2), (40, 128, 2), (1, 128, 2)])
def test_c5_stages_other_shapes(cuda, S, D, H):
    """Heads of 128 (RoPE tables [S, 64]) and sequence lengths off the
    16-query and 32-key blocks, one token included: the QKV + RoPE and
    attention stages against the oracle's stage values under the same
    bounds as the configuration's."""
    w = configs.llama_layer(S=S, D=D, H=H, F=128, seed=131 + S)
    inp = w.make_inputs()
    assert inp["cos_t"].shape == (S, D // H // 2)
    st = refs.llama_stages(inp, H, LL_EPS)
    ex = refs.llama_stage_exact(inp, st, H, LL_EPS)
    d = configs.to_device(inp)
    S, D = inp["x"].shape
    Q, K, V = _bf_dev((S, D)), _bf_dev((S, D)), _bf_dev((S, D))
    groups.fused_llama_qkv_rope(d["x"], d["g1"], d["wq"], d["wk"], d["wv"], d["cos_t"],
                                d["sin_t"], Q, K, V, LL_EPS)
    torch.cuda.synchronize()
    xn = refs.normed_bf16(inp["x"], inp["g1"], LL_EPS)
    for name, t, wname, rope in (("Q", Q, "wq", True), ("K", K, "wk", True), ("V", V, "wv", False)):
        mag = refs.mag_qkv(xn, inp[wname], inp["cos_t"], inp["sin_t"], rope)
        check_bf16_stage(_host(t), ex[name], mag, D + 2, what=f"{name} S={S} dh={D // H}")
    dq = configs.to_device({k: st[k] for k in ("Q", "K", "V")})
    A = _bf_dev((S, D))
    groups.fused_llama_attention(dq["Q"], dq["K"], dq["V"], A, H, (D // H) ** -0.5)
    torch.cuda.synchronize()
    mag = refs.mag_attention(st["Q"], st["K"], st["V"], H)
    check_bf16_stage(_host(A), ex["A"], mag, S + D // H, what=f"attention S={S} dh={D // H}")
    assert np.array_equal(_host(A)[0], st["V"][0])


def test_c5_stage_oproj_residual(cuda, llama_case):
    w, inp, st = llama_case
    d = configs.to_device({"A": st["A"], "wo": inp["wo"], "x": inp["x"]})
    h = _bf_dev(inp["x"].shape)
    groups.fused_llama_matmul_residual(d["A"], d["wo"], d["x"], h)
    torch.cuda.synchronize()
    mag = refs.mag_residual(st["A"], inp["wo"], inp["x"])
    check_bf16_rounded(_host(h), st["exact"]["h"], mag, inp["wo"].shape[0] + 1, what="h")


def test_c5_stage_swiglu(cuda, llama_case):
    w, inp, st = llama_case
    d = configs.to_device({"h": st["h"], "g2": inp["g2"], "wg": inp["wg"], "wu": inp["wu"]})
    act = _bf_dev(st["act"].shape)
    groups.fused_llama_rmsnorm_swiglu(d["h"], d["g2"], d["wg"], d["wu"], act, LL_EPS)
    torch.cuda.synchronize()
    hn = refs.normed_bf16(st["h"], inp["g2"], LL_EPS)
    mag = refs.mag_swiglu(hn, inp["wg"], inp["wu"])
    check_bf16_stage(_host(act), st["exact"]["act"], mag, inp["wg"].shape[0] + 4, what="act")


def test_c5_stage_down_residual(cuda, llama_case):
    w, inp, st = llama_case
    d = configs.to_device({"act": st["act"], "wd": inp["wd"], "h": st["h"]})
    out = _bf_dev(inp["x"].shape)
    groups.fused_llama_matmul_residual(d["act"], d["wd"], d["h"], out)
    torch.cuda.synchronize()
    mag = refs.mag_residual(st["act"], inp["wd"], st["h"])
    check_bf16_rounded(_host(out), st["exact"]["out"], mag, inp["wd"].shape[0] + 1, what="out")


def test_c5_layer_end_to_end(cuda, llama_case):
    w, inp, st = llama_case
    d = configs.to_device(inp)
    o = w.make_outputs(d)
    w.run(d, o, None)
    torch.cuda.synchronize()
    for name, (ref, mag) in refs.reference(w.name, inp).items():
        check_bound(bf16(_host(o[name])), bf16(ref), mag, RTOL_BF16, what=f"layer {name}")


# S = 1088: the last query block's 17 key blocks give each of the
# attention's four key groups five steps (an odd count), with K/V blocks
# refetched into both register slots on the way.  D = 448: the single-panel
# RMSNorm GEMMs with a half-filled last K chunk; D = 576: K past one panel,
# the general RMSNorm GEMM kernel.  F = 1088 and 1600: the down projection's
# K in three and four chunks (the last one ragged) through its two LDS
# buffers.
@pytest.mark.parametrize("S,D,H,F", [(64, 128, 2, 192), (128, 64, 1, 64), (96, 128, 2, 128),
                                     (1088, 128, 2, 128), (64, 448, 7, 128), (64, 576, 9, 192),
                                     (64, 128, 2, 1088), (32, 128, 2, 1600),
                                     # heads of 128 (the head dim is D / H)
                                     (64, 256, 2, 192), (96, 128, 1, 128), (256, 512, 4, 384),
                                     # sequence lengths off the 16- and 32-row blocks
                                     (40, 128, 2, 192), (17, 64, 1, 64), (100, 256, 2, 128),
                                     (1, 128, 2, 64)])
def test_c5_layer_small_shapes(cuda, S, D, H, F):
    w = configs.llama_layer(S=S, D=D, H=H, F=F, seed=91 + S)
    inp = w.make_inputs()
    d = configs.to_device(inp)
    o = w.make_outputs(d)
    groups.llama_layer(d, o, H, LL_EPS)
    torch.cuda.synchronize()
    for name, (ref, mag) in refs.llama_reference(inp, H, LL_EPS).items():
        check_bound(bf16(_host(o[name])), bf16(ref), mag, RTOL_BF16, what=f"layer {name}")


# ------------------------------------------------------------------ SRAM plan as LDS layout
def _planned_case(M, K, N, seed, bias=True):
    from npu_amd import tileplan
    A = rng.uniform(seed, 0, (M, K), -1, 1)
    B = rng.uniform(seed, 1, (K, N), -1, 1)
    b = rng.uniform(seed, 2, (N,), -1, 1) if bias else None
    text = blocks.matmul_bias_act(M, K, N, act="relu") if bias else None
    plan = tileplan.matmul_group_plan(mlir.parse_functions(text)[0])
    return A, B, b, plan


@pytest.mark.parametrize("M,K,N", [(256, 512, 256), (100, 36, 52), (64, 1000, 80)])
def test_planned_matmul_layout_is_the_plan(cuda, M, K, N):
    """The group run as the reference's tile loop with its SRAM plan as the
    LDS layout: the output within the f32 bound of the oracle, and tile
    (0, 0)'s LDS holding each slice at its planned offset -- the bias slice,
    the last K step's A and B slices in the buffer of that step's parity,
    the accumulator tile and the output tile, which is what was stored."""
    A, B, b, p = _planned_case(M, K, N, 40 + M)
    plan = p["plan"]
    tm, tn, tk = p["tile"]
    out = torch.empty((M, N), dtype=torch.float32, device="cuda")
    dump = torch.zeros(plan.lds_bytes // 4, dtype=torch.float32, device="cuda")
    groups.planned_matmul_bias_act(_dev(A), _dev(B), _dev(b), out, plan, "relu", lds_dump=dump)
    torch.cuda.synchronize()
    ref, mag = refs.matmul_bias_act(A, B, b, "relu")
    got = _host(out)
    check_bound(got, ref, mag, RTOL_F32, what="planned matmul")
    lds = _host(dump)
    at = lambda off, rows, cols: lds[off // 4: off // 4 + rows * cols].reshape(rows, cols)
    mt, nt = min(tm, M), min(tn, N)
    assert np.array_equal(at(plan.off_bias, 1, tn)[0, :nt], b[:nt].astype(np.float32))
    nk = -(-K // tk)
    last = (nk - 1) % 2
    k0 = (nk - 1) * tk
    a_last = at(plan.off_a_pong if last else plan.off_a, tm, tk)
    b_last = at(plan.off_b_pong if last else plan.off_b, tk, tn)
    kk = min(tk, K - k0)
    assert np.array_equal(a_last[:mt, :kk], A[:mt, k0:k0 + kk].astype(np.float32))
    assert not a_last[:mt, kk:].any()  # K past the operand: zeros
    assert np.array_equal(b_last[:kk, :nt], B[k0:k0 + kk, :nt].astype(np.float32))
    c = at(plan.off_c, tm, tn)[:mt, :nt]
    r0, m0 = refs.matmul_bias_act(A[:mt], B[:, :nt], None, "none")
    check_bound(c, r0, m0, RTOL_F32, what="accumulator tile in SRAM")
    assert np.array_equal(at(plan.off_y, tm, tn)[:mt, :nt], got[:mt, :nt])


def test_planned_matmul_relu_mlir_closed_form(cuda):
    """test/matmul_relu.mlir (the builder's text of it, checked against the
    reference's file on the CPU) under the harness's rules (f16 -> f32,
    argument i filled with 0.01 (i + 1)) through its own plan: every output
    is K * 0.01 * 0.02 = 0.0512 (e2e_verify.py:288-309)."""
    from npu_amd import tileplan
    f = mlir.parse_functions(lower.harness_f32(blocks.reference_workload("matmul_relu.mlir")))[0]
    p = tileplan.matmul_group_plan(f)
    (na, ta), (nb, tb) = f.args[:2]
    A = torch.full(ta.shape, 0.01, dtype=torch.float32, device="cuda")
    B = torch.full(tb.shape, 0.02, dtype=torch.float32, device="cuda")
    out = torch.empty((ta.shape[0], tb.shape[1]), dtype=torch.float32, device="cuda")
    groups.planned_matmul_bias_act(A, B, None, out, p["plan"], "relu")
    torch.cuda.synchronize()
    got = _host(out)
    assert np.allclose(got, ta.shape[1] * 0.01 * 0.02, rtol=1e-5, atol=1e-7)


def _conv_plan_case(shape, bias, seed):
    from npu_amd import tileplan
    N, Cc, F, H, W = shape
    text = (blocks.nchw_conv_bias_act(N, Cc, F, H, W, act="relu6") if bias
            else lower.harness_f32(blocks.nchw_conv_relu(N, Cc, F, H, W)))
    p = tileplan.conv_group_plan(mlir.parse_functions(text)[0])
    x = rng.uniform(seed, 0, (N, Cc, H, W), -1, 1)
    w = rng.uniform(seed, 1, (F, Cc, 3, 3), -1, 1)
    b = rng.uniform(seed, 2, (F,), -1, 1) if bias else None
    return p, oracle.pad_nchw(x, (1, 1, 1, 1)), w, b


# (shape N, C, F, H, W; bias): the layouts the reference's plan gives them
PLANNED_CONV = [
    ((1, 64, 64, 56, 56), False),   # conv2d_relu.mlir: rows ping/pong/prefetch, filters spilled
    ((2, 5, 45, 64, 19), True),     # 3 tiles, the last ragged; every input with a prefetch region
    ((1, 4, 64, 90, 15), True),     # 4 tiles: tile i+2 fetched into the prefetch regions
    ((1, 64, 96, 112, 20), True),   # filters' ping only, rows without a prefetch region
    ((1, 128, 64, 56, 56), False),  # rows' ping only, filters spilled, 4 tiles
    ((1, 256, 64, 56, 56), False),  # rows and filters spilled, one tile
    ((1, 8, 20, 40, 16), True),     # one tile of all 20 channels
]


@pytest.mark.parametrize("shape,bias", PLANNED_CONV, ids=lambda v: "x".join(map(str, v))
                         if isinstance(v, tuple) else ("bias" if v else "nobias"))
def test_planned_conv_layout_is_the_plan(cuda, shape, bias):
    """The conv group run as the reference's tile loop over output-channel
    tiles with its SRAM plan as the LDS layout: the output within the f32
    bound of the oracle (relu6 with a bias, relu without), and workgroup
    0's LDS (image 0, output row 0) holding each slice at its planned
    offset: the input rows in every slot the loop filled, the last tile's
    filter and bias slices in the buffer of that tile's parity, the tile
    before it in the other, the last tile's copy in the prefetch regions
    (zeros past F), the accumulator row and the output row, which is what
    was stored."""
    p, xp, w, b = _conv_plan_case(shape, bias, 70 + shape[1])
    plan = p["plan"]
    N, Cc, F, H, W = shape
    tco, nt = p["tco"], p["tiles"]
    print(f"planned conv {shape} tco {tco} tiles {nt}", flush=True)
    out = torch.empty((N, F, H, W), dtype=torch.float32, device="cuda")
    dump = torch.zeros(plan.lds_bytes // 4, dtype=torch.float32, device="cuda")
    act = "relu6" if bias else "relu"
    groups.planned_conv2d_nchw_bias_act(_dev(xp), _dev(w), _dev(b), out, plan, act, lds_dump=dump)
    torch.cuda.synchronize()
    ref, mag = refs.conv_nchw_act(xp, w, b, pad=0, act=act)
    got = _host(out)
    check_bound(got, ref, mag, RTOL_F32, what=f"planned conv {shape}")
    lds = _host(dump)
    at = lambda off, n: lds[off // 4: off // 4 + n]
    rows = xp[0, :, 0:3, :].astype(np.float32).ravel()
    filled = [plan.off_in] + ([plan.off_in_pong, plan.off_in_prefetch] if nt > 1 else [])
    for off in filled:
        if off >= 0:
            assert np.array_equal(at(off, rows.size), rows)

    def slice_of(t, arr, per):
        v = np.zeros((tco,) + arr.shape[1:], np.float32)
        f0 = t * tco
        v[:max(0, min(tco, F - f0))] = arr[f0:f0 + tco]
        return v.ravel()

    last, prev = nt - 1, nt - 2
    for arr, ping, pong, pre in ((w, plan.off_w, plan.off_w_pong, plan.off_w_prefetch),
                                 (b, plan.off_bias, plan.off_bias_pong, plan.off_bias_prefetch)):
        if arr is None or ping < 0:
            continue
        slots = [ping, pong if pong >= 0 else ping]
        want = slice_of(last, arr, None)
        assert np.array_equal(at(slots[last & 1], want.size), want)
        if nt > 1 and pong >= 0:
            wp = slice_of(prev, arr, None)
            assert np.array_equal(at(slots[prev & 1], wp.size), wp)
        if nt > 1 and pre >= 0:
            assert np.array_equal(at(pre, want.size), want)
    nl = min(tco, F - last * tco)
    c = at(plan.off_c, tco * W).reshape(tco, W)[:nl]
    r0, m0 = refs.conv_nchw_act(xp[:1, :, 0:3], w[last * tco:last * tco + nl], None, pad=0,
                                act="none")
    check_bound(c, r0[0, :, 0], m0[0, :, 0], RTOL_F32, what="accumulator row in SRAM")
    y = at(plan.off_y, tco * W).reshape(tco, W)[:nl]
    assert np.array_equal(y, got[0, last * tco:last * tco + nl, 0])


# ------------------------------------------------------------------ host lowering
@pytest.mark.parametrize("case", ["matmul", "conv_f32", "conv_bf16", "inverted_residual",
                                  "inverted_residual_64x384"])
def test_lowered_blocks_match_the_oracle(cuda, case):
    """linalg text -> npu_amd.lower -> entry-point calls on the GPU, against
    the oracle of the same block."""
    if case == "matmul":
        A = rng.uniform(15, 0, (64, 96), -1, 1)
        B = rng.uniform(15, 1, (96, 48), -1, 1)
        b = rng.uniform(15, 2, (48,), -1, 1)
        prog = lower.lower_text(blocks.matmul_bias_act(64, 96, 48, act="relu6"))
        out = prog.run({"A": _dev(A), "B": _dev(B), "bias": _dev(b)})["%y"]
        torch.cuda.synchronize()
        ref, mag = refs.matmul_bias_act(A, B, b, "relu6")
        check_bound(_host(out), ref, mag, RTOL_F32, what="lowered matmul")
    elif case.startswith("conv"):
        elem = "bf16" if case == "conv_bf16" else "f32"
        x = rng.uniform(16, 0, (2, 9, 7, 32), 0, 1)
        w = rng.normal(16, 1, (64, 3, 3, 32), 0, math.sqrt(2 / (9 * 32)))
        b = rng.uniform(16, 2, (64,), -0.1, 0.1)
        if elem == "bf16":
            # every argument in its declared type: the bias too (the group
            # widens it to f32 exactly and adds in f32)
            x, w, b = rng.to_bf16_bits(x), rng.to_bf16_bits(w), rng.to_bf16_bits(b)
        prog = lower.lower_text(blocks.conv_bias_act(2, 9, 7, 32, 64, elem=elem))
        out = prog.run({"x": _dev(x), "w": _dev(w), "bias": _dev(b)})["%y"]
        torch.cuda.synchronize()
        bias32 = bf16(b).astype(np.float32) if elem == "bf16" else b
        ref, mag = refs.conv_bias_act(x, w, bias32, 1, "relu")
        if elem == "f32":
            check_bound(_host(out), ref, mag, RTOL_F32, what="lowered conv")
        else:
            ref32, _ = _widened_conv(x, w, bias32, 1, "relu")
            check_bf16_rounded(_host(out), ref32, mag, 9 * 32 + 1, what="lowered conv")
    else:
        # the configuration's channels, and a MobileNetV2 block the streaming
        # kernel runs
        N, H, W, C, E = (2, 9, 13, 24, 144) if case == "inverted_residual" else (1, 14, 14, 64, 384)
        x = rng.uniform(17, 0, (N, H, W, C), 0, 1)
        we = rng.normal(17, 1, (E, C), 0, math.sqrt(2 / C))
        wdw = rng.normal(17, 2, (3, 3, E), 0, math.sqrt(2 / 9))
        wp = rng.normal(17, 3, (C, E), 0, math.sqrt(2 / E))
        prog = lower.lower_text(blocks.inverted_residual(N, H, W, C, E))
        assert prog.entry_points == ["fused_irb_f32"]
        out = prog.run({"x": _dev(x), "we": _dev(we.reshape(E, 1, 1, C)), "wdw": _dev(wdw),
                        "wp": _dev(wp.reshape(C, 1, 1, E))})["%y"]
        torch.cuda.synchronize()
        ref, mag = refs.irb(x, we, wdw, wp)
        check_bound(_host(out), ref, mag, RTOL_F32, what="lowered inverted residual")


# ------------------------------------------------------------------ reference workloads
def _harness_fills(prog):
    """The reference harness's argument fills: argument i holds 0.01 * (i + 1)
    (tools/harness/e2e_verify.py:186-203)."""
    ins = {}
    for i, (a, t) in enumerate(prog.func.args):
        ins[a] = torch.full(t.shape, 0.01 * (i + 1), dtype=torch.float32, device="cuda")
    return ins


@pytest.mark.parametrize("name", ["matmul_relu.mlir", "mlp.mlir"])
def test_reference_workloads_run_on_the_gpu(cuda, name):
    """test/matmul_relu.mlir and test/mlp.mlir (the builder's text of them,
    checked against the reference's files on the CPU), f16 run as f32 the way
    the harness runs them, with the harness's fills, through the lowering and
    npu_group_launch: the closed forms 0.0512 (K = 256) and
    512 * 0.0512 * 0.03 = 0.786432, and the oracle's unfused loops."""
    prog = lower.lower_text(blocks.reference_workload(name))
    ins = _harness_fills(prog)
    (res,) = prog.run(ins).values()
    torch.cuda.synchronize()
    got = _host(res).astype(np.float64)
    host_ins = [_host(ins[a]) for a, _ in prog.func.args]
    if name == "matmul_relu.mlir":
        assert np.all(np.abs(got - 0.0512) <= 1e-4 * 0.0512)
        ref = oracle.block_matmul_bias_act(host_ins[0], host_ins[1], None, "relu")
    else:
        assert len(prog.launches) == 1 and [c.entry for c in prog.calls] == \
            ["fused_matmul_bias_act"] * 2
        assert np.all(np.abs(got - 0.786432) <= 1e-5 * 0.786432 * 2)
        h = oracle.block_matmul_bias_act(host_ins[0], host_ins[1], None, "relu")
        ref = oracle.block_matmul_bias_act(h, host_ins[2], None, "relu")
    assert np.all(np.abs(got - ref) <= 1e-5 * np.abs(ref) * 2)


NCHW_WORKLOADS = ["conv2d_relu.mlir", "resnet_block.mlir", "resnet50_block.mlir",
                  "mobilenet_block.mlir"]


@pytest.mark.parametrize("fills", ["harness", "seeded"])
@pytest.mark.parametrize("name", NCHW_WORKLOADS)
def test_reference_nchw_workloads_run_on_the_gpu(cuda, name, fills):
    """The reference's own conv workloads -- linalg.conv_2d_nchw_fchw groups
    outlined as @fused_fill_conv2d_generic[_generic]_<idx>, f16 run as f32 --
    lowered and launched group by group through npu_group_launch (the pads
    folded, the ResNet adds as residual terms), against the oracle's unfused
    NCHW loops: with the harness's fills 0.01 (i + 1) (e2e_verify.py:186-203)
    and with seeded inputs (U(0, 1) activations, He-normal filters)."""
    prog = lower.lower_text(blocks.reference_workload(name))
    if fills == "harness":
        ins = _harness_fills(prog)
    else:
        ins = {}
        for i, (a, t) in enumerate(prog.func.args):
            if i == 0:
                arr = rng.uniform(31, i, tuple(t.shape), 0, 1)
            else:
                fan = int(np.prod(t.shape[1:]))
                arr = rng.normal(31, i, tuple(t.shape), 0, math.sqrt(2 / fan))
            ins[a] = _dev(arr)
    (res,) = prog.run(ins).values()
    torch.cuda.synchronize()
    host_ins = [_host(ins[a]) for a, _ in prog.func.args]
    with oracle.threaded():
        ref, mag = refs.nchw_workload(name, host_ins)
    check_bound(_host(res), ref, mag, RTOL_F32, what=f"{name} ({fills})")
    assert all(L.name.startswith("fused_fill_conv2d_generic") for L in prog.launches)


@pytest.mark.parametrize("N,C,H,W,F,K,pad,st,act,bias,res", [
    (2, 20, 9, 37, 40, 3, 1, 1, "relu", True, False),    # C and F off the 16 / 64 blocks, ragged segments
    (1, 64, 56, 56, 64, 3, 1, 1, "relu", False, True),   # the reference's conv, with a residual
    (1, 256, 14, 14, 64, 1, 0, 1, "relu6", True, False),  # 1x1, sixteen channel chunks
    (3, 8, 5, 70, 24, 3, 0, 1, "none", False, True),     # valid conv, rows past one segment
    (1, 192, 28, 112, 192, 3, 1, 1, "relu", False, False),  # 64-pixel segments (large grid)
    (1, 4, 3, 3, 4, 1, 0, 1, "none", True, False),       # a handful of values
    (2, 64, 15, 15, 128, 3, 1, 2, "relu", True, True),   # stride 2, odd sizes (staged kernel)
    (1, 64, 14, 14, 128, 1, 0, 2, "none", False, False),  # the 1x1 stride-2 shortcut
    (1, 3, 30, 34, 64, 7, 3, 2, "relu", False, False),   # a 7x7/2 stem (direct kernel)
    (1, 32, 9, 9, 40, 5, 2, 1, "relu6", True, False),    # 5x5 (direct)
    (1, 20, 11, 13, 24, 9, 4, 1, "relu", False, True),   # 9x9, pad 4 (direct)
    (1, 512, 7, 7, 100, 7, 0, 1, "none", False, False),  # the classifier as a conv: 1x1 output
])
def test_nchw_conv_shapes(cuda, N, C, H, W, F, K, pad, st, act, bias, res):
    x = rng.uniform(32, 0, (N, C, H, W), -1, 1)
    w = rng.normal(32, 1, (F, C, K, K), 0, math.sqrt(2 / (K * K * C)))
    b = rng.uniform(32, 2, (F,), -0.1, 0.1) if bias else None
    Ho, Wo = (H + 2 * pad - K) // st + 1, (W + 2 * pad - K) // st + 1
    r = rng.uniform(32, 3, (N, F, Ho, Wo), -1, 1) if res else None
    out = torch.empty(N, F, Ho, Wo, device="cuda")
    if res:
        groups.fused_conv2d_nchw_bias_res_act(_dev(x), _dev(w), None if b is None else _dev(b),
                                              _dev(r), out, pad, act, stride=st)
    else:
        groups.fused_conv2d_nchw_bias_act(_dev(x), _dev(w), None if b is None else _dev(b), out,
                                          pad, act, stride=st)
    torch.cuda.synchronize()
    ref, mag = refs.conv_nchw_act(x, w, b, r, pad, act, stride=st)
    check_bound(_host(out), ref, mag, RTOL_F32,
                what=f"nchw conv {N}x{C}x{H}x{W} -> {F} {K}x{K}/{st}")


def test_nchw_conv_non_finite(cuda):
    """NaN and +-Inf through the NCHW conv on the f32 matrix pipe: the same
    positions and values as the oracle's f32 loops."""
    N, C, H, W, F = 1, 32, 12, 20, 32
    x = rng.uniform(33, 0, (N, C, H, W), 0, 1)
    x[0, 3, 4, 5] = np.nan
    x[0, 7, 9, 15] = np.inf
    w = rng.normal(33, 1, (F, C, 3, 3), 0, 0.1)
    out = torch.empty(N, F, H, W, device="cuda")
    groups.fused_conv2d_nchw_bias_act(_dev(x), _dev(w), None, out, 1, "none")
    torch.cuda.synchronize()
    got = _host(out)
    ref, mag = refs.conv_nchw_act(x, w, None, None, 1, "none")
    hit = ~np.isfinite(ref)
    assert hit.sum() > 9 * F
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = hit & ~np.isnan(ref)
    assert np.array_equal(got[fin], ref[fin])
    check_bound(got[~hit], ref[~hit], mag[~hit], RTOL_F32, what="nchw conv next to NaN / Inf")


@pytest.mark.parametrize("name", ["resnet18", "resnet50", "vgg11", "srcnn", "espcn",
                                  "dcgan_generator", "autoencoder", "autoencoder_deep"])
def test_model_zoo_networks_run_on_the_gpu(cuda, name):
    """Whole networks of the reference's model zoo (test/models/<name>.mlir,
    the builder's text, checked op for op against the file on the CPU), f16
    run as f32: lowered, every group launched through npu_group_launch or,
    for a group of two conv chains (a ResNet downsampling block's shortcut
    and second conv), its entry points; U(0, 1) input, He-normal weights.
    Every launch's result is held to the f32 bound against the oracle's loops
    run on that launch's own inputs (the GPU's results of the launches
    before it); the network's output is within a relative 2-norm of 1e-4 of
    the oracle run end to end (f32 rounding through up to 50 layers stays
    near 1e-6; a wrong layout, stride, pad or residual gives order 1).  The
    element-wise magnitude bound end to end would be vacuous here: |W|
    products grow far faster than the values through the layers."""
    from npu_amd import model_zoo
    prog = lower.lower_text(model_zoo.model(name))
    ins, host = {}, []
    for i, (a, t) in enumerate(prog.func.args):
        if i == 0:
            arr = rng.uniform(34, i, tuple(t.shape), 0, 1)
        else:
            fan = int(np.prod(t.shape[1:])) if len(t.shape) == 4 else t.shape[0]
            arr = rng.normal(34, i, tuple(t.shape), 0, math.sqrt(2 / fan))
        host.append(arr)
        ins[a] = _dev(arr)
    print(f"{name}: {len(prog.launches)} launches", flush=True)
    vals = prog.check_inputs(ins)
    for li in range(len(prog.launches)):
        prog.run_launch(li, vals)
    torch.cuda.synchronize()
    gpu = {v: _host(t) for v, t in vals.items() if v not in ins and v.lstrip("%") not in ins}
    with oracle.threaded():
        per, mags, _ = refs.run_network(prog.func, host, given=gpu)
        end, _, depth = refs.run_network(prog.func, host)
    for L in prog.launches:
        for v in L.outs or [L.out]:
            check_bound(gpu[v], per[v], mags[v], RTOL_F32, what=f"{name}: launch {L.name} -> {v}")
    (out,) = [op.operands[0] for op in prog.func.ops if op.name == "func.return"]
    rel = np.linalg.norm(gpu[out].astype(np.float64) - end[out]) / np.linalg.norm(end[out])
    print(f"{name}: depth {depth[out]}, end-to-end relative 2-norm {rel:.3g}", flush=True)
    assert rel <= 1e-4, f"{name}: end-to-end relative difference {rel:.3g}"


def test_int8_frontend_runs_on_the_gpu(cuda):
    """A float ResNet bottleneck (C = 256, M1 = 64) quantized by the int8
    frontend, lowered and run: bit-exact against the oracle's int8 loops."""
    import torch.nn as nn
    from test_frontend import _FloatBottleneck
    torch.manual_seed(2)
    m = _FloatBottleneck(C=256, M=64, bn=True)
    with torch.no_grad():
        for c in (m.c1, m.c2, m.c3):
            nn.init.kaiming_normal_(c.weight)
    x = torch.rand(4, 256, 14, 14)
    text, a = frontend.from_torch_int8(m, x)
    prog = lower.lower_text(text)
    (res,) = prog.run({k: configs.to_device({k: v})[k] for k, v in a.items()}).values()
    torch.cuda.synchronize()
    ref = oracle.block_qbottleneck(a["x"], a["w1"].reshape(64, 256), a["w2"],
                                   a["w3"].reshape(256, 64), a["m1"], a["s1"], a["m2"], a["s2"],
                                   a["m3"], a["s3"])
    assert np.array_equal(_host(res), ref)


def test_bf16_frontend_runs_on_the_gpu(cuda):
    """The torch frontend in bf16: a BasicBlock (conv, batch norm folded,
    ReLU, conv, batch norm, residual, ReLU) traced to bf16 NHWC linalg,
    lowered (biases widened to f32) and run, against the block computed in
    float64 from the same bf16 arguments, stage bound (the first conv's
    output is rounded to bf16 before the second conv reads it)."""
    import torch.nn as nn
    from test_frontend import BasicBlock, randomize_bn
    torch.manual_seed(3)
    m = randomize_bn(BasicBlock(64))
    x = torch.rand(2, 64, 14, 14)
    text, params = frontend.from_torch(m, x, elem="bf16", name="basic_bf16")
    prog = lower.lower_text(text)
    dev = {k: v.cuda() for k, v in params.items()}
    (res,) = prog.run(dev).values()
    torch.cuda.synchronize()
    f = {k: v.double() for k, v in params.items()}
    y1 = torch.relu(torch.nn.functional.conv2d(f["x0"].permute(0, 3, 1, 2),
                                               f["w1"].permute(0, 3, 1, 2), f["b2"], padding=1))
    y1 = y1.to(torch.bfloat16).double()
    out = torch.nn.functional.conv2d(y1, f["w3"].permute(0, 3, 1, 2), f["b4"], padding=1) + \
        f["x0"].permute(0, 3, 1, 2)
    exact = torch.relu(out).permute(0, 2, 3, 1).numpy()
    a = lambda t: t.abs()
    m1 = torch.nn.functional.conv2d(a(f["x0"]).permute(0, 3, 1, 2), a(f["w1"]).permute(0, 3, 1, 2),
                                    a(f["b2"]), padding=1)
    mag = (torch.nn.functional.conv2d(m1, a(f["w3"]).permute(0, 3, 1, 2), a(f["b4"]), padding=1) +
           a(f["x0"]).permute(0, 3, 1, 2)).permute(0, 2, 3, 1).numpy()
    got = _host(res)
    check_bf16_stage(got, exact, mag, 9 * 64 + 2, what="bf16 BasicBlock")


def test_compiled_c_caller_on_the_gpu(cuda):
    """The C program that calls npu_group_launch by outlined name with MLIR
    memref descriptors: the matmul_relu and mlp closed forms and the C1 group
    with a bias against the oracle."""
    import os
    import subprocess
    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c", "group_launch_test")
    print("running", exe, "gpu", flush=True)
    r = subprocess.run([exe, "gpu"], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr


COST_KEYS = ["name", "flops", "mem_bytes", "arithmetic_intensity", "time_sec", "is_memory_bound",
             "efficiency", "dma_in_bytes", "dma_out_bytes", "matrix_cycles", "dsp_cycles",
             "peak_sram_bytes", "num_tile_iterations", "num_linalg_ops", "sram_budget", "bottleneck"]


@pytest.mark.parametrize("which", ["mlp", "irb", "llama"])
def test_cost_records_carry_prediction_and_measurement(cuda, which):
    """COST_JSON records of a lowered program: the reference's keys in its
    order (CostEvaluatePass.cpp:135-158), then the entry point, the MI355X
    launch model's prediction and the measured device time of that launch;
    summed like tools/harness/optimize.py:73-94 sums time_sec."""
    import json
    if which == "mlp":
        prog = lower.lower_text(blocks.reference_workload("mlp.mlir"))
        ins = _harness_fills(prog)
    elif which == "llama":
        prog = lower.lower_text(blocks.llama_layer(128, 256, 4, 512))
        ins = _llama_text_inputs(configs.llama_layer(S=128, D=256, H=4, F=512).make_inputs())
    else:
        N, H, W, C, E = 2, 9, 13, 24, 144
        prog = lower.lower_text(blocks.inverted_residual(N, H, W, C, E))
        ins = {"x": _dev(rng.uniform(17, 0, (N, H, W, C), 0, 1)),
               "we": _dev(rng.normal(17, 1, (E, 1, 1, C), 0, 0.3)),
               "wdw": _dev(rng.normal(17, 2, (3, 3, E), 0, 0.5)),
               "wp": _dev(rng.normal(17, 3, (C, 1, 1, E), 0, 0.1))}
    lines = lower.cost_report(prog, ins, reps=10)
    recs = [json.loads(line[len("COST_JSON: "):]) for line in lines]
    assert len(recs) == sum(len(L.name.split("+")) for L in prog.launches)
    for r in recs:
        assert list(r)[:len(COST_KEYS)] == COST_KEYS
        assert list(r)[len(COST_KEYS):] == ["entry_point", "mi355x_predicted_us", "measured_us"]
        assert r["mi355x_predicted_us"] > 0 and r["measured_us"] > 0
    total_measured = sum({r["entry_point"]: r["measured_us"] for r in recs}.values())
    print("measured", total_measured, "predicted",
          sum({r["entry_point"]: r["mi355x_predicted_us"] for r in recs}.values()))


def _llama_text_inputs(inp):
    d = configs.to_device(inp)
    d["cos"], d["sin"] = d.pop("cos_t"), d.pop("sin_t")
    return d


@pytest.mark.parametrize("S,D,H,F", [(64, 128, 2, 192), (256, 512, 8, 1408), (64, 256, 2, 192)])
def test_lowered_llama_layer_matches_the_oracle(cuda, S, D, H, F):
    """The Llama layer's linalg text through the lowering: five calls of the
    Llama entry points, bit-identical to calling them directly, and within
    the bf16 bound of the oracle's layer."""
    w = configs.llama_layer(S=S, D=D, H=H, F=F, seed=77 + S)
    inp = w.make_inputs()
    prog = lower.lower_text(blocks.llama_layer(S, D, H, F))
    vals = prog.run(_llama_text_inputs(inp))
    d = configs.to_device(inp)
    o = w.make_outputs(d)
    groups.llama_layer(d, o, H, LL_EPS)
    torch.cuda.synchronize()
    assert np.array_equal(_host(vals["%out"]), _host(o["out"]))
    ref, mag = refs.llama_reference(inp, H, LL_EPS)["out"]
    check_bound(bf16(_host(vals["%out"])), bf16(ref), mag, RTOL_BF16, what="lowered layer")


@pytest.mark.parametrize("N,H,W,C", [(2, 7, 9, 64), (1, 12, 10, 256)])
def test_lowered_int8_bottleneck_is_bit_exact(cuda, N, H, W, C):
    """The int8 bottleneck's linalg text (apply_scale requant generics, pad,
    residual) through the lowering and npu_group_launch: bit-exact against
    the oracle's unfused loops."""
    w = configs.qbottleneck(N, H=H, W=W, C=C, M1=64)
    a = w.make_inputs()
    prog = lower.lower_text(blocks.qbottleneck(N, H, W, C, 64))
    ins = {k: _dev(v) for k, v in a.items()}
    ins["w1"] = ins["w1"].reshape(64, 1, 1, C)
    ins["w3"] = ins["w3"].reshape(C, 1, 1, 64)
    (out,) = prog.run(ins).values()
    torch.cuda.synchronize()
    ref = refs.qbottleneck(a)
    assert np.array_equal(_host(out), ref)


# ------------------------------------------------------------------ frontends
def _f64_nchw(t):
    return t.double().permute(0, 3, 1, 2)


@pytest.mark.parametrize("which", ["basic_block", "inverted_residual", "mlp"])
def test_torch_frontend_runs_on_the_gpu(cuda, which):
    """A torch module traced to NHWC linalg (npu_amd.frontend), lowered and run
    on the GPU, against the module itself in float64 on the CPU.  The bound
    is 1e-5 of the chain's magnitude per contraction stage (each stage's f32
    error scales with its own magnitude and passes through the later stages'
    linear maps, which the magnitude recursion bounds)."""
    import torch.nn.functional as Fn
    from test_frontend import MLP, BasicBlock, InvertedResidual, randomize_bn
    torch.manual_seed(7)
    if which == "basic_block":
        m, x = randomize_bn(BasicBlock(64)), torch.rand(4, 64, 14, 14)
    elif which == "inverted_residual":
        m, x = InvertedResidual(24, 144), torch.rand(2, 24, 28, 28)
    else:
        m, x = MLP(256, 512, 128), torch.rand(64, 256) - 0.5
    import copy
    text, params = frontend.from_torch(m, x)
    prog = lower.lower_text(text)
    (out,) = prog.run({k: v.cuda() for k, v in params.items()}).values()
    torch.cuda.synchronize()
    got = out.double().cpu()
    p = {k: v.double() for k, v in params.items()}
    with torch.no_grad():
        ref = copy.deepcopy(m).double()(x.double())
    if which == "basic_block":
        ref = ref.permute(0, 2, 3, 1)
        a = lambda t: t.abs()
        m1 = Fn.conv2d(_f64_nchw(a(p["x0"])), a(p["w1"]).permute(0, 3, 1, 2), a(p["b2"]), padding=1)
        mag = Fn.conv2d(m1, a(p["w3"]).permute(0, 3, 1, 2), a(p["b4"]), padding=1) + _f64_nchw(a(p["x0"]))
        mag, stages = mag.permute(0, 2, 3, 1), 2
    elif which == "inverted_residual":
        ref = ref.permute(0, 2, 3, 1)
        xa = _f64_nchw(p["x0"].abs())
        me = Fn.conv2d(xa, p["w1"].abs().permute(0, 3, 1, 2))
        md = Fn.conv2d(me, p["w2"].abs().permute(2, 0, 1).unsqueeze(1), padding=1, groups=144)
        mag = (Fn.conv2d(md, p["w3"].abs().permute(0, 3, 1, 2)) + xa).permute(0, 2, 3, 1)
        stages = 3
    else:
        m1 = p["x0"].abs() @ p["w1"].abs() + p["b2"].abs()
        mag, stages = m1 @ p["w3"].abs() + p["b4"].abs(), 2
    check_bound(got.numpy(), ref.numpy(), mag.numpy(), stages * RTOL_F32, what=which)


@pytest.mark.parametrize("C,M,final_relu", [(24, 144, False), (256, 64, True)])
def test_model_zoo_block_runs_on_the_gpu(cuda, C, M, final_relu):
    """Residual blocks in the reference's model-zoo form (NCHW, f16 text:
    test/models/mobilenetv2.mlir:166-226's inverted residual block,
    resnet50.mlir:194-267's bottleneck; written by
    blocks.model_zoo_bottleneck), run the way the reference's harness runs its
    texts (f16 -> f32) after the NCHW -> NHWC rewrite, against torch's float64
    NCHW convolutions of the same data."""
    import torch.nn.functional as Fn
    N, H, W = 2, 56, 56
    f = mlir.parse_functions(lower.harness_f32(
        blocks.model_zoo_bottleneck(N, C, M, H, W, final_relu)))[0]
    prog = lower.lower(frontend.nchw_to_nhwc(f))
    g = torch.Generator().manual_seed(11 + C)
    x = torch.rand(N, C, H, W, generator=g)
    w1 = torch.randn(M, C, 1, 1, generator=g) * (2 / C) ** 0.5
    w2 = torch.randn(M, M, 3, 3, generator=g) * (2 / (9 * M)) ** 0.5
    w3 = torch.randn(C, M, 1, 1, generator=g) * (2 / M) ** 0.5
    nhwc = lambda t: t.permute(0, 2, 3, 1).contiguous().cuda()
    (out,) = prog.run({"x": nhwc(x), "w1": nhwc(w1), "w2": nhwc(w2), "w3": nhwc(w3)}).values()
    torch.cuda.synchronize()
    xd, d1, d2, d3 = x.double(), w1.double(), w2.double(), w3.double()
    r1 = Fn.relu(Fn.conv2d(xd, d1))
    r2 = Fn.relu(Fn.conv2d(r1, d2, padding=1))
    ref = Fn.conv2d(r2, d3) + xd
    ref = (Fn.relu(ref) if final_relu else ref).permute(0, 2, 3, 1)
    m1 = Fn.conv2d(xd.abs(), d1.abs())
    m2 = Fn.conv2d(m1, d2.abs(), padding=1)
    mag = (Fn.conv2d(m2, d3.abs()) + xd.abs()).permute(0, 2, 3, 1)
    check_bound(out.double().cpu().numpy(), ref.numpy(), mag.numpy(), 3 * RTOL_F32,
                what=f"model-zoo block C={C} M={M}")


@pytest.mark.parametrize("N,H,W,C,F,dtype", [(2, 9, 13, 24, 40, "f32"), (1, 7, 7, 48, 24, "bf16")])
def test_conv_residual_and_odd_channels(cuda, N, H, W, C, F, dtype):
    """fused_conv2d_nhwc_bias_res_act with channel counts that are not a
    multiple of an MFMA fragment (C = 24, 48; F = 40, 24), against the
    oracle's conv plus the residual."""
    x = rng.uniform(41, 0, (N, H, W, C), 0, 1)
    w = rng.normal(41, 1, (F, 3, 3, C), 0, math.sqrt(2 / (9 * C)))
    b = rng.uniform(41, 2, (F,), -0.1, 0.1)
    r = rng.uniform(41, 3, (N, H, W, F), -1, 1)
    ref, mag = refs.conv_bias_act(x, w, b, 1, "none")
    want = np.maximum(ref.astype(np.float64) + r, 0.0)
    mag = mag + np.abs(r)
    if dtype == "bf16":
        xb, wb, rb = rng.to_bf16_bits(x), rng.to_bf16_bits(w), rng.to_bf16_bits(r)
        ref32, mag = refs.conv_bias_act(bf16(xb).astype(np.float32), bf16(wb).astype(np.float32), b, 1,
                                        "none")
        want = np.maximum(ref32.astype(np.float64) + bf16(rb), 0.0)
        mag = mag + np.abs(bf16(rb))
        out = torch.empty(N, H, W, F, device="cuda", dtype=torch.bfloat16)
        groups.fused_conv2d_nhwc_bias_res_act(_dev(xb), _dev(wb), _dev(b), _dev(rb), out, 1, "relu")
        torch.cuda.synchronize()
        check_bf16_rounded(_host(out), want, mag, 9 * C + 2, what="bf16 conv + residual")
    else:
        out = torch.empty(N, H, W, F, device="cuda", dtype=torch.float32)
        groups.fused_conv2d_nhwc_bias_res_act(_dev(x), _dev(w), _dev(b), _dev(r), out, 1, "relu")
        torch.cuda.synchronize()
        check_bound(_host(out), want, mag, RTOL_F32, what="f32 conv + residual")
