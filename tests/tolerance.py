"""Per-element error bounds used by the parity tests.

fp32 and bf16 results are compared in the error-bound form
    |gpu - oracle| <= rtol * mag + atol
where ``mag`` is the same expression evaluated on absolute values
(sum_k |a_k * b_k| + |bias| ... propagated through the chain).  A different
summation order (MFMA, split-K) changes a sum of n terms by at most about
n * eps * mag, so the bound is independent of cancellation in the result.
rtol is 1e-5 for fp32 paths and 2e-2 for bf16 paths.  Integer paths are
compared bit for bit.

A bf16 result rounded once, from an f32 accumulation of n products of the
same bf16 inputs on both sides, is held to the rounding-aware bound of
``check_bf16_rounded``, against the oracle's f32 value of the chain before that
rounding (the f32 loops over the widened inputs, which form the same exact
products in the same order):
    |gpu - oracle_f32| <= 2^-8 (1 + 2^-7) |oracle_f32| + 2 n 2^-23 mag
(the two f32 sums differ by at most 2 n 2^-24 mag; the GPU's one
round-to-nearest-even to bf16 adds at most 2^-8 of its value).  It is far
tighter than 2e-2 mag: a dropped product larger than about 2^-8 of the result
is outside it.

The Llama sub-groups are held to ``check_bf16_stage``, against the stage's
value computed in float64 from the same bf16 inputs:
    |gpu - exact| <= 2^-8 (1 + 2^-7) |exact| + (2^-8 + 2 n 2^-23) mag
The extra 2^-8 mag is what the GPU may legitimately do differently inside
the stage: the RMSNorm stages normalise the rows themselves (a different sum
order and reciprocal square root can move a normalised bf16 input by one
unit in the last place, 2^-8 of it, so the products by at most 2^-8 mag), and
attention rounds the softmax probabilities to bf16 before P.V (2^-9 of each
term, so at most 2^-9 mag) and uses the hardware exponential.  That is five
times tighter than 2e-2 mag.
"""
import numpy as np

RTOL_F32 = 1e-5
RTOL_BF16 = 2e-2


def check_bound(gpu, ref, mag, rtol, atol=0.0, what=""):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    mag = np.asarray(mag, np.float64)
    assert gpu.shape == ref.shape == mag.shape, (gpu.shape, ref.shape, mag.shape)
    assert np.all(np.isfinite(gpu)), f"{what}: non-finite GPU output"
    err = np.abs(gpu - ref)
    bound = rtol * mag + atol
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {err.size} elements outside rtol={rtol} bound; "
            f"worst at {i}: gpu={gpu[i]!r} ref={ref[i]!r} mag={mag[i]!r} err={err[i]:.3e}")
    return float((err / np.maximum(mag, 1e-30)).max())


def bf16(x):
    """bf16 bit patterns -> float64 values."""
    x = np.ascontiguousarray(x, np.uint16)
    return (x.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def check_bf16_rounded(gpu_bits, ref_f32, mag, n_terms, what=""):
    """The rounding-aware bf16 bound (module docstring): bf16 bit patterns
    against the oracle's f32 value before its rounding."""
    g, r = bf16(gpu_bits), np.asarray(ref_f32, np.float64)
    mag = np.asarray(mag, np.float64)
    assert g.shape == r.shape == mag.shape, (g.shape, r.shape, mag.shape)
    assert np.all(np.isfinite(g)), f"{what}: non-finite GPU output"
    err = np.abs(g - r)
    bound = 2.0 ** -8 * (1 + 2.0 ** -7) * np.abs(r) + 2 * n_terms * 2.0 ** -23 * mag
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {err.size} elements outside the bf16 rounding bound; "
            f"worst at {i}: gpu={g[i]!r} ref={r[i]!r} mag={mag[i]!r} err={err[i]:.3e}")
    return float((err / np.maximum(np.abs(r) + mag, 1e-30)).max())


def check_bf16_stage(gpu_bits, exact, mag, n_terms, what=""):
    """The Llama stage bound (module docstring): bf16 bit patterns against the
    stage's float64 value."""
    g, r = bf16(gpu_bits), np.asarray(exact, np.float64)
    mag = np.asarray(mag, np.float64)
    assert g.shape == r.shape == mag.shape, (g.shape, r.shape, mag.shape)
    assert np.all(np.isfinite(g)), f"{what}: non-finite GPU output"
    err = np.abs(g - r)
    bound = 2.0 ** -8 * (1 + 2.0 ** -7) * np.abs(r) + (2.0 ** -8 + 2 * n_terms * 2.0 ** -23) * mag
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {err.size} elements outside the bf16 stage bound; "
            f"worst at {i}: gpu={g[i]!r} ref={r[i]!r} mag={mag[i]!r} err={err[i]:.3e}")
    return float((err / np.maximum(np.abs(r) + mag, 1e-30)).max())
