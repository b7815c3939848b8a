"""Pins the CPU restatement (oracle/) before anything is compared against it.

Three kinds of checks, per the oracle function they cover:
  * the reference harness's own known-answer tests (tests/golden/reference_kats.json,
    written by tests/golden/make_reference_kats.py from
    tools/harness/{e2e_verify,numerical_verify,verify_accuracy}.py);
  * library routines evaluated independently in float64 (torch conv2d,
    numpy matmul/pad, torch's bf16 rounding, Python big integers);
  * invariants the mathematics fixes (M-tiling is bit-exact, RoPE at
    position 0 is the identity and preserves pair norms, softmax rows sum to 1).
Inputs are random, non-square and non-symmetric so that a transposed operand,
a wrong index or a dropped term fails; the ``planted`` tests show the checks
reject exactly such mistakes.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import oracle
from npu_amd import inputs as rng
from tolerance import RTOL_BF16, bf16, check_bound

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))["cases"]
EPS32 = 2.0 ** -24


def kat(name):
    return next(c for c in KATS if c["name"] == name)


def gamma(n):
    """Higham's gamma_n = n*u / (1 - n*u) for binary32."""
    return n * EPS32 / (1 - n * EPS32)


def r32(seed, shape, lo=-1.0, hi=1.0):
    return rng.uniform(seed, 7, shape, lo, hi)


# ------------------------------------------------------------ reference KATs
@pytest.mark.parametrize("name", ["e2e_matmul_relu", "e2e_matmul_relu_k512"])
def test_kat_e2e_matmul_relu(name):
    c = kat(name)
    A = np.full((c["M"], c["K"]), c["fill_a"], np.float32)
    B = np.full((c["K"], c["N"]), c["fill_b"], np.float32)
    out = oracle.block_matmul_bias_act(A, B, None, "relu")
    np.testing.assert_allclose(out, c["expected_value"], atol=c["atol"], rtol=c["rtol"])
    assert abs(out[0, 0] - c["K"] * 0.01 * 0.02) < c["atol"]


@pytest.mark.parametrize("c", [k for k in KATS if k["kind"] == "matmul_tiled"],
                         ids=lambda c: c["name"])
def test_kat_numerical_matmul_tiled(c):
    A = np.full((c["M"], c["K"]), c["fill_a"], np.float32)
    B = np.full((c["K"], c["N"]), c["fill_b"], np.float32)
    orig = oracle.matmul(A, B)
    tiled = oracle.matmul_tiled_m(A, B, c["tile_m"])
    np.testing.assert_allclose(orig, c["expected_value"], atol=c["atol"], rtol=0)
    np.testing.assert_allclose(tiled, c["expected_value"], atol=c["atol"], rtol=0)
    assert np.max(np.abs(orig - tiled)) <= c["atol_orig_vs_tiled"]


def test_kat_numerical_conv2d():
    c = kat("numerical_conv2d_1x2x6x6_2x2x3x3")
    x = np.full(c["input_shape"], c["fill_input"], np.float32)
    w = np.full(c["filter_shape"], c["fill_filter"], np.float32)
    out = oracle.conv2d_nchw_fchw(x, w)
    assert out.shape == tuple(c["output_shape"])
    np.testing.assert_allclose(out, c["expected_value"], atol=c["atol"], rtol=0)
    np.testing.assert_allclose(out, 0.0036, atol=c["atol"], rtol=0)


def test_kat_numerical_relu():
    c = kat("numerical_relu_4x4")
    out = oracle.relu(np.full(c["shape"], c["fill"], np.float32))
    np.testing.assert_allclose(out, c["expected_value"], atol=c["atol"])


def test_kat_verify_accuracy_matmul_ktiled():
    c = kat("verify_accuracy_matmul_ktiled")
    g = np.random.default_rng(42)
    A = (g.standard_normal((c["M"], c["K"])) * 0.1).astype(np.float32)
    B = (g.standard_normal((c["K"], c["N"])) * 0.1).astype(np.float32)
    full = oracle.matmul(A, B)
    acc = np.zeros((c["M"], c["N"]), np.float32)
    for k in range(0, c["K"], c["tile_k"]):
        acc = oracle.matmul(np.ascontiguousarray(A[:, k:k + c["tile_k"]]),
                            np.ascontiguousarray(B[k:k + c["tile_k"]]), acc)
    assert np.max(np.abs(full - acc)) < c["abs_threshold"]
    np.testing.assert_allclose(np.max(np.abs(full)), c["max_abs_ref"], rtol=1e-5)


def test_kat_verify_accuracy_relu_tiled():
    c = kat("verify_accuracy_relu_tiled")
    x = (np.random.default_rng(42).standard_normal(c["shape"]) * 0.5).astype(np.float32)
    whole = oracle.relu(x)
    tiled = np.concatenate([oracle.relu(x[i:i + c["tile"]]) for i in range(0, len(x), c["tile"])])
    assert np.array_equal(whole, tiled)
    assert np.array_equal(whole, np.maximum(x, 0))


# ------------------------------------------------------------ matmul family
def test_matmul_vs_float64():
    A, B = r32(1, (7, 33)), rng.uniform(2, 3, (33, 5), -1, 1)
    C = oracle.matmul(A, B)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    mag = np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)
    assert np.all(np.abs(C - ref) <= gamma(33) * mag)


def test_matmul_accumulates_into_init():
    A, B = r32(3, (4, 6)), r32(4, (6, 3))
    C0 = r32(5, (4, 3))
    C = oracle.matmul(A, B, C0)
    ref = C0.astype(np.float64) + A.astype(np.float64) @ B.astype(np.float64)
    assert np.allclose(C, ref, atol=1e-5)


def test_matmul_tiled_m_bit_exact_random():
    A, B = r32(6, (13, 17)), r32(7, (17, 9))
    assert np.array_equal(oracle.matmul(A, B), oracle.matmul_tiled_m(A, B, 4))


def test_batch_matmul_vs_float64():
    A, B = r32(8, (3, 5, 7)), r32(9, (3, 7, 4))
    C = oracle.batch_matmul(A, B)
    ref = np.einsum("bmk,bkn->bmn", A.astype(np.float64), B.astype(np.float64))
    assert np.allclose(C, ref, atol=1e-5)


def test_matmul_bf16_is_exact_products():
    A = rng.to_bf16_bits(r32(10, (6, 40)))
    B = rng.to_bf16_bits(r32(11, (40, 3)))
    C = oracle.matmul_bf16(A, B)
    ref = bf16(A) @ bf16(B)
    mag = np.abs(bf16(A)) @ np.abs(bf16(B))
    assert np.all(np.abs(C - ref) <= gamma(40) * mag)


def test_planted_transposed_operand_is_caught():
    """A square matmul with B transposed must fail the same bound."""
    A, B = r32(12, (16, 16)), r32(13, (16, 16))
    wrong = oracle.matmul(A, np.ascontiguousarray(B.T))
    ref = A.astype(np.float64) @ B.astype(np.float64)
    mag = np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)
    assert not np.all(np.abs(wrong - ref) <= 1e-5 * mag)


# ------------------------------------------------------------ elementwise
def test_relu_relu6_add_bias_silu():
    x = r32(14, (5, 8), -8, 8)
    assert np.array_equal(oracle.relu(x), np.maximum(x, 0))
    assert np.array_equal(oracle.relu6(x), np.minimum(np.maximum(x, 0), 6))
    y = r32(15, (5, 8))
    assert np.array_equal(oracle.add(x, y), x + y)
    b = r32(16, (8,))
    assert np.array_equal(oracle.bias_add(x, b), x + b[None, :])
    g, u = r32(17, (40,), -6, 6), r32(18, (40,))
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(oracle.silu_mul(g, u), ref, rtol=1e-6, atol=1e-7)


def test_relu_propagates_nan():
    x = np.array([np.nan, -1.0, 2.0], np.float32)
    r = oracle.relu(x)
    assert np.isnan(r[0]) and r[1] == 0 and r[2] == 2


def test_pad_matches_numpy():
    x = r32(19, (2, 3, 4, 5))
    assert np.array_equal(oracle.pad_nhwc(x, (1, 2, 0, 1)),
                          np.pad(x, ((0, 0), (1, 2), (0, 1), (0, 0))))
    assert np.array_equal(oracle.pad_nchw(x, (1, 1, 1, 1)),
                          np.pad(x, ((0, 0), (0, 0), (1, 1), (1, 1))))
    xi = rng.randint(1, 2, (1, 3, 3, 4), -128, 127).astype(np.int8)
    assert np.array_equal(oracle.pad_nhwc(xi, (1, 1, 1, 1)),
                          np.pad(xi, ((0, 0), (1, 1), (1, 1), (0, 0))))


# ------------------------------------------------------------ convolutions
def _torch_conv_nhwc(x, w, pad=0, groups=1):
    xt = torch.from_numpy(np.asarray(x, np.float64)).permute(0, 3, 1, 2)
    wt = torch.from_numpy(np.asarray(w, np.float64))
    o = torch.nn.functional.conv2d(xt, wt, padding=pad, groups=groups)
    return o.permute(0, 2, 3, 1).numpy()


def test_conv_nchw_vs_torch():
    x, w = r32(20, (2, 3, 7, 6)), r32(21, (4, 3, 3, 2))
    out = oracle.conv2d_nchw_fchw(x, w)
    ref = torch.nn.functional.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double())
    mag = torch.nn.functional.conv2d(torch.from_numpy(np.abs(x)).double(),
                                     torch.from_numpy(np.abs(w)).double())
    assert np.all(np.abs(out - ref.numpy()) <= gamma(18) * mag.numpy())


def test_conv_nhwc_vs_torch_and_stride():
    x, w = r32(22, (2, 9, 8, 6)), r32(23, (5, 3, 3, 6))
    out = oracle.conv2d_nhwc_fhwc(x, w)
    ref = _torch_conv_nhwc(x, w.transpose(0, 3, 1, 2))
    mag = _torch_conv_nhwc(np.abs(x), np.abs(w).transpose(0, 3, 1, 2))
    assert np.all(np.abs(out - ref) <= gamma(54) * mag)
    out2 = oracle.conv2d_nhwc_fhwc(x, w, stride=(2, 2))
    assert np.allclose(out2, ref[:, ::2, ::2, :], atol=1e-5)


def test_conv_nhwc_bf16_and_i8():
    x, w = r32(24, (1, 6, 5, 8)), r32(25, (4, 3, 3, 8))
    xb, wb = rng.to_bf16_bits(x), rng.to_bf16_bits(w)
    out = oracle.conv2d_nhwc_fhwc(xb, wb)
    ref = _torch_conv_nhwc(bf16(xb), bf16(wb).transpose(0, 3, 1, 2))
    mag = _torch_conv_nhwc(np.abs(bf16(xb)), np.abs(bf16(wb)).transpose(0, 3, 1, 2))
    assert np.all(np.abs(out - ref) <= gamma(72) * mag)
    xi = rng.randint(3, 0, (1, 6, 5, 8), -128, 127)
    wi = rng.randint(3, 1, (4, 3, 3, 8), -127, 127)
    outi = oracle.conv2d_nhwc_fhwc(xi.astype(np.int8), wi.astype(np.int8))
    refi = np.zeros((1, 4, 3, 4), np.int64)
    for kh in range(3):
        for kw in range(3):
            refi += np.einsum("nhwc,fc->nhwf", xi[:, kh:kh + 4, kw:kw + 3, :], wi[:, kh, kw, :])
    assert np.array_equal(outi, refi)


def test_depthwise_vs_torch_grouped():
    x, w = r32(26, (2, 7, 6, 5)), r32(27, (3, 3, 5))
    out = oracle.depthwise_conv2d_nhwc_hwc(x, w)
    wt = w.transpose(2, 0, 1)[:, None, :, :]  # [C,1,KH,KW]
    ref = _torch_conv_nhwc(x, wt, groups=5)
    mag = _torch_conv_nhwc(np.abs(x), np.abs(wt), groups=5)
    assert np.all(np.abs(out - ref) <= gamma(9) * mag)


def test_planted_flipped_filter_is_caught():
    x, w = r32(28, (1, 6, 6, 4)), r32(29, (3, 3, 3, 4))
    wrong = oracle.conv2d_nhwc_fhwc(x, np.ascontiguousarray(w[:, ::-1, ::-1, :]))
    ref = _torch_conv_nhwc(x, w.transpose(0, 3, 1, 2))
    mag = _torch_conv_nhwc(np.abs(x), np.abs(w).transpose(0, 3, 1, 2))
    assert not np.all(np.abs(wrong - ref) <= 1e-5 * mag)


# ------------------------------------------------------------ bf16 rounding
def test_bf16_round_to_nearest_even_matches_torch():
    specials = np.array([0.0, -0.0, 1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9,
                         -(1.0 + 2 ** -8), 3.3895314e38, np.inf, -np.inf, 1e-40, -1e-45,
                         65504.0, 2 ** -126], np.float32)
    x = np.concatenate([specials, rng.normal(30, 0, (4000,), 0, 100)])
    ours = oracle.trunc_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.array_equal(ours, rng.to_bf16_bits(x))
    assert np.array_equal(oracle.ext_bf16(ours), bf16(ours).astype(np.float32))
    nan = oracle.trunc_bf16(np.array([np.nan], np.float32))
    assert np.isnan(bf16(nan)[0])


# ------------------------------------------------------------ integer requant
def _apply_scale_py(acc, m, s):
    return (int(acc) * int(m) + (1 << (int(s) - 1))) >> int(s)


def test_apply_scale_vs_big_integers():
    acc = rng.randint(40, 0, (64, 8), -(2 ** 23), 2 ** 23).astype(np.int32)
    acc[0, :] = [0, 1, -1, 2 ** 22, -(2 ** 22), 3, -3, 7]
    mult = rng.randint(40, 1, (8,), 2 ** 30, 2 ** 31 - 1).astype(np.int32)
    shift = np.array([31, 32, 35, 38, 40, 45, 50, 55], np.int32)
    out = oracle.apply_scale(acc, mult, shift)
    for i in range(acc.shape[0]):
        for c in range(8):
            assert out[i, c] == _apply_scale_py(acc[i, c], mult[c], shift[c])


def test_apply_scale_rounds_half_up():
    # (acc * m) / 2^s = x.5 exactly: single round adds 2^(s-1) then floors.
    m, s = np.array([1 << 30], np.int32), np.array([31], np.int32)
    acc = np.array([[1], [-1], [3], [-3]], np.int32)  # 0.5, -0.5, 1.5, -1.5
    out = oracle.apply_scale(acc, m, s).ravel().tolist()
    assert out == [1, 0, 2, -1]


def test_clamp_i8():
    x = np.array([-300, -1, 0, 5, 127, 128, 999], np.int32)
    assert oracle.clamp_i8(x, 0, 127).tolist() == [0, 0, 0, 5, 127, 127, 127]
    assert oracle.clamp_i8(x, -128, 127).tolist() == [-128, -1, 0, 5, 127, 127, 127]


# ------------------------------------------------------------ norms / rope / softmax
def test_rmsnorm_vs_float64():
    x, g = r32(41, (6, 64), -3, 3), r32(42, (64,), 0.5, 1.5)
    out = oracle.rmsnorm(x, g, 1e-5)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-5) * g
    np.testing.assert_allclose(out, ref, rtol=2e-6, atol=1e-7)


def _rope_tables(S, Dh, theta=10000.0):
    inv = theta ** (-np.arange(0, Dh, 2, dtype=np.float64) / Dh)
    ang = np.arange(S, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def test_rope_identity_norm_and_complex_rotation():
    S, H, Dh = 5, 2, 8
    x = r32(43, (S, H * Dh))
    c, s = _rope_tables(S, Dh)
    out = oracle.rope(x, c, s, H)
    assert np.array_equal(out[0], x[0])  # position 0: cos 1, sin 0
    xp = x.reshape(S, H, Dh // 2, 2).astype(np.float64)
    op = out.reshape(S, H, Dh // 2, 2).astype(np.float64)
    np.testing.assert_allclose(np.hypot(op[..., 0], op[..., 1]), np.hypot(xp[..., 0], xp[..., 1]),
                               rtol=1e-6)
    z = (xp[..., 0] + 1j * xp[..., 1]) * (c.astype(np.float64) + 1j * s)[:, None, :]
    np.testing.assert_allclose(op[..., 0], z.real, atol=1e-6)
    np.testing.assert_allclose(op[..., 1], z.imag, atol=1e-6)


def test_causal_softmax_vs_float64():
    s = r32(44, (6, 9), -4, 4)
    p = oracle.causal_softmax(s)
    off = 9 - 6
    sd = s.astype(np.float64)
    for i in range(6):
        vis = sd[i, :i + off + 1]
        e = np.exp(vis - vis.max())
        np.testing.assert_allclose(p[i, :i + off + 1], e / e.sum(), rtol=2e-6, atol=1e-8)
        assert np.all(p[i, i + off + 1:] == 0)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-6)


# ------------------------------------------------------------ composite blocks
def test_block_matmul_bias_relu_vs_float64():
    A, B, b = r32(50, (20, 36)), r32(51, (36, 12)), r32(52, (12,))
    out = oracle.block_matmul_bias_act(A, B, b, "relu")
    ref = np.maximum(A.astype(np.float64) @ B + b, 0)
    mag = np.abs(A).astype(np.float64) @ np.abs(B) + np.abs(b)
    assert np.all(np.abs(out - ref) <= gamma(40) * mag)


def test_block_conv_bias_relu_f32_and_bf16():
    x = rng.uniform(53, 0, (2, 7, 5, 16), 0, 1)
    w = rng.normal(53, 1, (8, 3, 3, 16), 0, math.sqrt(2 / 144))
    b = rng.uniform(53, 2, (8,), -0.1, 0.1)
    out = oracle.block_conv_bias_act(x, w, b, 1, "relu")
    ref = np.maximum(_torch_conv_nhwc(x, w.transpose(0, 3, 1, 2), pad=1) + b, 0)
    mag = _torch_conv_nhwc(np.abs(x), np.abs(w).transpose(0, 3, 1, 2), pad=1) + np.abs(b)
    assert np.all(np.abs(out - ref) <= gamma(150) * mag)
    xb, wb = rng.to_bf16_bits(x), rng.to_bf16_bits(w)
    outb = oracle.block_conv_bias_act(xb, wb, b, 1, "relu")
    refb = np.maximum(_torch_conv_nhwc(bf16(xb), bf16(wb).transpose(0, 3, 1, 2), pad=1) + b, 0)
    # one bf16 rounding of the result (2^-9 relative) on top of f32 accumulation
    assert np.all(np.abs(bf16(outb) - refb) <= 2 ** -8 * np.abs(refb) + gamma(150) * mag)


def test_block_irb_vs_float64():
    x = rng.uniform(54, 0, (2, 6, 5, 8), 0, 1)
    we = rng.normal(54, 1, (24, 8), 0, math.sqrt(2 / 8))
    wdw = rng.normal(54, 2, (3, 3, 24), 0, math.sqrt(2 / 9))
    wp = rng.normal(54, 3, (8, 24), 0, math.sqrt(2 / 24))
    out = oracle.block_irb(x, we, wdw, wp)
    xd = x.astype(np.float64)
    e = np.clip(np.einsum("nhwc,ec->nhwe", xd, we), 0, 6)
    d = np.clip(_torch_conv_nhwc(e, wdw.transpose(2, 0, 1)[:, None], pad=1, groups=24), 0, 6)
    ref = np.einsum("nhwe,ce->nhwc", d, wp) + xd
    me = np.einsum("nhwc,ec->nhwe", np.abs(xd), np.abs(we))
    md = _torch_conv_nhwc(me, np.abs(wdw).transpose(2, 0, 1)[:, None], pad=1, groups=24)
    mag = np.einsum("nhwe,ce->nhwc", md, np.abs(wp)) + np.abs(xd)
    assert np.all(np.abs(out - ref) <= 1e-5 * mag)


def _requant_np(acc, m, s):
    acc = acc.astype(np.int64)
    return (acc * m.astype(np.int64) + (np.int64(1) << (s.astype(np.int64) - 1))) >> s.astype(np.int64)


def test_block_qbottleneck_vs_int64():
    N, H, W, Cc, M1 = 2, 5, 6, 32, 16
    x = rng.randint(55, 0, (N, H, W, Cc), 0, 127)
    w1 = rng.randint(55, 1, (M1, Cc), -127, 127)
    w2 = rng.randint(55, 2, (M1, 3, 3, M1), -127, 127)
    w3 = rng.randint(55, 3, (Cc, M1), -127, 127)
    m = [rng.randint(55, 4 + i, (n,), 2 ** 30, 2 ** 31 - 1) for i, n in enumerate((M1, M1, Cc))]
    s = [np.full((n,), sh, np.int64) for n, sh in ((M1, 44), (M1, 45), (Cc, 44))]
    out = oracle.block_qbottleneck(x.astype(np.int8), w1, w2, w3, m[0], s[0], m[1], s[1], m[2], s[2])
    y1 = np.clip(_requant_np(np.einsum("nhwc,fc->nhwf", x, w1), m[0], s[0]), 0, 127)
    y1p = np.pad(y1, ((0, 0), (1, 1), (1, 1), (0, 0)))
    a2 = np.zeros((N, H, W, M1), np.int64)
    for kh in range(3):
        for kw in range(3):
            a2 += np.einsum("nhwc,fc->nhwf", y1p[:, kh:kh + H, kw:kw + W], w2[:, kh, kw])
    y2 = np.clip(_requant_np(a2, m[1], s[1]), 0, 127)
    ref = np.clip(_requant_np(np.einsum("nhwc,fc->nhwf", y2, w3), m[2], s[2]) + x, 0, 127)
    assert np.array_equal(out.astype(np.int64), ref)
    assert 0 < np.count_nonzero(y1) < y1.size  # the chosen scales exercise both clamp sides


def _bf(x):
    return torch.from_numpy(np.asarray(x, np.float64)).to(torch.bfloat16).double()


def test_block_llama_layer_vs_float64():
    S, D, H, F, eps = 16, 32, 2, 48, 1e-5
    Dh = D // H
    f = lambda i, shape, sd: rng.to_bf16_bits(rng.normal(56, i, shape, 0, sd))
    x = f(0, (S, D), 1.0)
    wq, wk, wv, wo = (f(i, (D, D), 0.2) for i in (1, 2, 3, 4))
    wg, wu, wd = f(5, (D, F), 0.2), f(6, (D, F), 0.2), f(7, (F, D), 0.2)
    g1, g2 = rng.uniform(56, 8, (D,), 0.5, 1.5), rng.uniform(56, 9, (D,), 0.5, 1.5)
    c, s = _rope_tables(S, Dh)
    h, out = oracle.block_llama_layer(x, g1, g2, wq, wk, wv, wo, wg, wu, wd, c, s, H, eps)
    # float64 reference with the same bf16 rounding points
    T = lambda a: torch.from_numpy(bf16(a))
    xd = T(x)

    def rms(v, g):
        return v / torch.sqrt((v * v).mean(-1, keepdim=True) + eps) * torch.from_numpy(g).double()

    def rope_t(v):
        vv = v.reshape(S, H, Dh // 2, 2)
        z = torch.complex(vv[..., 0], vv[..., 1]) * torch.complex(
            torch.from_numpy(c).double(), torch.from_numpy(s).double())[:, None, :]
        return torch.stack([z.real, z.imag], -1).reshape(S, D)

    xn = _bf(rms(xd, g1))
    Q, K, V = _bf(rope_t(xn @ T(wq))), _bf(rope_t(xn @ T(wk))), _bf(xn @ T(wv))
    q4, k4, v4 = (t.reshape(S, H, Dh).transpose(0, 1) for t in (Q, K, V))
    sc = (q4 @ k4.transpose(1, 2)) / math.sqrt(Dh)
    sc = sc.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    A = _bf((torch.softmax(sc, -1) @ v4).transpose(0, 1).reshape(S, D))
    href = _bf(xd + A @ T(wo))
    hn = _bf(rms(href, g2))
    g = hn @ T(wg)
    act = _bf(g / (1 + torch.exp(-g)) * (hn @ T(wu)))
    oref = _bf(href + act @ T(wd))
    magh = (xd.abs() + A.abs() @ T(wo).abs()).numpy()
    mago = (href.abs() + act.abs() @ T(wd).abs()).numpy()
    check_bound(bf16(h), href.numpy(), magh, RTOL_BF16, what="h")
    check_bound(bf16(out), oref.numpy(), mago, RTOL_BF16, what="out")


# ------------------------------------------------------------ the OpenMP build
@pytest.mark.parametrize("which", ["matmul", "conv_f32", "conv_bf16", "irb", "qbottleneck",
                                   "llama"])
def test_threaded_oracle_returns_the_same_bits(which):
    """The all-cores CPU baseline runs libnpu_oracle_omp.so: the same loops
    with the outer parallel loops split over threads.  Every output must be
    bit-identical to the single-threaded checker's."""
    import refs
    from npu_amd import configs
    w = {"matmul": lambda: configs.matmul_bias_relu(64, 128, 32),
         "conv_f32": lambda: configs.conv3x3_bias_relu(2, "f32", H=7, W=9, C=16, F=16),
         "conv_bf16": lambda: configs.conv3x3_bias_relu(2, "bf16", H=7, W=9, C=32, F=16),
         "irb": lambda: configs.irb(2, H=6, W=5),
         "qbottleneck": lambda: configs.qbottleneck(2, H=6, W=7, C=64, M1=64),
         "llama": lambda: configs.llama_layer(S=64, D=128, H=2, F=256)}[which]()
    inp = w.make_inputs()
    name = w.name
    if which == "llama":
        old = refs.LLAMA_HEADS
        refs.LLAMA_HEADS = 2
    try:
        serial = refs.run_oracle(name, inp)
        with oracle.threaded():
            par = refs.run_oracle(name, inp)
    finally:
        if which == "llama":
            refs.LLAMA_HEADS = old
    for k in serial:
        assert np.array_equal(np.asarray(serial[k]), np.asarray(par[k])), k


def test_bf16_conv_is_the_widened_f32_chain_rounded_once():
    """The bf16 GPU checks compare against the oracle's f32 value before its
    final rounding, computed as the f32 chain over the widened inputs: that
    value rounded to bf16 must be the bf16 oracle's output bit for bit."""
    import refs
    x = rng.to_bf16_bits(rng.uniform(60, 0, (2, 7, 9, 32), 0, 1))
    w = rng.to_bf16_bits(rng.normal(60, 1, (16, 3, 3, 32), 0, math.sqrt(2 / 288)))
    b = rng.uniform(60, 2, (16,), -0.1, 0.1)
    outb = oracle.block_conv_bias_act(x, w, b, 1, "relu")
    ref32, _ = refs.conv_bias_act(bf16(x).astype(np.float32), bf16(w).astype(np.float32), b, 1,
                                  "relu")
    assert np.array_equal(rng.to_bf16_bits(ref32), outb)


def test_bf16_rounding_bound_rejects_one_dropped_channel_of_one_tap():
    """Planted mistake at the full C2 bf16 shape (one image): the chain with
    channel 5 of tap (1, 1) dropped, rounded to bf16, fails the rounding-aware
    bound the GPU test applies, while the correct chain rounded passes."""
    import refs
    from npu_amd import configs
    from tolerance import check_bf16_rounded
    wl = configs.conv3x3_bias_relu(1, "bf16")
    a = wl.make_inputs()
    xf, wf = bf16(a["x"]).astype(np.float32), bf16(a["w"]).astype(np.float32)
    ref32, mag = refs.conv_bias_act(xf, wf, a["bias"], 1, "relu")
    check_bf16_rounded(rng.to_bf16_bits(ref32), ref32, mag, 9 * 64 + 1, what="correct")
    w_bad = wf.copy()
    w_bad[:, 1, 1, 5] = 0.0
    bad32, _ = refs.conv_bias_act(xf, w_bad, a["bias"], 1, "relu")
    with pytest.raises(AssertionError, match="outside the bf16 rounding bound"):
        check_bf16_rounded(rng.to_bf16_bits(bad32), ref32, mag, 9 * 64 + 1, what="planted")


def test_llama_stage_bound_accepts_the_oracle_and_rejects_dropped_terms():
    """The Llama stage bound the GPU tests apply: the oracle's own sub-group
    outputs pass it against the float64 stage values, and planted mistakes
    fail it: a 1 % gain on the down projection's and on attention's output,
    which the 2e-2 bound lets through."""
    import refs
    from npu_amd import configs
    from tolerance import check_bf16_rounded, check_bf16_stage
    H, eps = 2, 1e-5
    w = configs.llama_layer(S=64, D=128, H=H, F=192, seed=5)
    inp = w.make_inputs()
    st = refs.llama_stages(inp, H, eps)
    ex = refs.llama_stage_exact(inp, st, H, eps)
    xn = refs.normed_bf16(inp["x"], inp["g1"], eps)
    hn = refs.normed_bf16(st["h"], inp["g2"], eps)
    for name, wname, rope in (("Q", "wq", True), ("K", "wk", True), ("V", "wv", False)):
        mag = refs.mag_qkv(xn, inp[wname], inp["cos_t"], inp["sin_t"], rope)
        check_bf16_stage(st[name], ex[name], mag, 128 + 2, what=name)
    check_bf16_stage(st["A"], ex["A"], refs.mag_attention(st["Q"], st["K"], st["V"], H), 64 + 64,
                     what="A")
    m_h = refs.mag_residual(st["A"], inp["wo"], inp["x"])
    check_bf16_rounded(st["h"], ex["h"], m_h, 128 + 1, what="h")
    check_bf16_stage(st["act"], ex["act"], refs.mag_swiglu(hn, inp["wg"], inp["wu"]), 128 + 4,
                     what="act")
    m_out = refs.mag_residual(st["act"], inp["wd"], st["h"])
    check_bf16_rounded(st["out"], ex["out"], m_out, 192 + 1, what="out")
    # planted: a 1 % gain on the output (inside 2e-2 mag, since mag >= |out|)
    bad = rng.to_bf16_bits(bf16(st["out"]) * 1.01)
    check_bound(bf16(bad), bf16(st["out"]), m_out, RTOL_BF16, what="2e-2 lets it through")
    with pytest.raises(AssertionError, match="bf16 rounding bound"):
        check_bf16_rounded(bad, ex["out"], m_out, 192 + 1, what="planted")
    # planted: a 1 % gain on attention's output
    badA = rng.to_bf16_bits(bf16(st["A"]) * 1.01)
    m_a = refs.mag_attention(st["Q"], st["K"], st["V"], H)
    check_bound(bf16(badA), bf16(st["A"]), m_a, RTOL_BF16, what="2e-2 lets it through")
    with pytest.raises(AssertionError, match="bf16 stage bound"):
        check_bf16_stage(badA, ex["A"], m_a, 128, what="planted A")
