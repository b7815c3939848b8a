"""GPU parity of the fused-group kernels against the CPU restatement.

Every call goes through the C-ABI (npu_amd.groups -> libnpu_amd.so).  fp32
results must lie within rtol 1e-5 and bf16 within rtol 2e-2 of the oracle in
the error-bound form of tests/tolerance.py; integer results bit for bit.
Configuration sizes run in full where the oracle takes seconds; batch-32
runs check a subset of images of the full-size launch against the oracle
(images are independent), plus size-independent properties.
"""
import math

import numpy as np
import pytest
import torch

import oracle
import refs
from npu_amd import configs, groups
from npu_amd import inputs as rng
from tolerance import RTOL_BF16, RTOL_F32, bf16, check_bound

pytestmark = pytest.mark.gpu


def _dev(a):
    return configs.to_device({"a": a})["a"]


def _host(t):
    return configs.to_host(t)


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
        check_bound(bf16(out["out"]), bf16(ref), mag, RTOL_BF16, what=w.name)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_c2_conv_config_n32(cuda, dtype):
    w = configs.conv3x3_bias_relu(32, dtype)
    arrs, out = _run_workload(w)
    imgs = [0, 17, 31]
    ref, mag = refs.reference(w.name, arrs, images=imgs)["out"]
    got = out["out"][imgs]
    if dtype == "f32":
        check_bound(got, ref, mag, RTOL_F32, what=w.name)
    else:
        check_bound(bf16(got), bf16(ref), mag, RTOL_BF16, what=w.name)
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
        check_bound(bf16(_host(out)), bf16(ref), mag, RTOL_BF16, what="conv")


def test_c2_reference_kat_fills(cuda):
    """numerical_verify's conv closed form (fills 0.01/0.02, unpadded) at C=16:
    every output is C*KH*KW*0.01*0.02."""
    x = torch.full((1, 6, 6, 16), 0.01, device="cuda")
    w = torch.full((16, 3, 3, 16), 0.02, device="cuda")
    out = torch.empty(1, 4, 4, 16, device="cuda")
    groups.fused_conv2d_nhwc_bias_act(x, w, None, out, 0, "none")
    np.testing.assert_allclose(_host(out), 16 * 9 * 0.01 * 0.02, atol=1e-5)
