"""Per-element error bounds used by the parity tests.

fp32 and bf16 results are compared in the error-bound form
    |gpu - oracle| <= rtol * mag + atol
where ``mag`` is the same expression evaluated on absolute values
(sum_k |a_k * b_k| + |bias| ... propagated through the chain).  A different
summation order (MFMA, split-K) changes a sum of n terms by at most about
n * eps * mag, so the bound is independent of cancellation in the result.
rtol is 1e-5 for fp32 paths and 2e-2 for bf16 paths.  Integer paths are
compared bit for bit.
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
