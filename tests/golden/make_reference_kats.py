"""Write reference_kats.json: the known-answer tests the reference's harness holds.

The reference pins CPU-executed linalg with constant-fill inputs.  Each case
below records the inputs the harness builds, the expected output the harness
compares against (its numpy closed form, evaluated here the same way, in
numpy float32) and the tolerance it applies.  Sources:

* tools/harness/e2e_verify.py:186-205, 274-279, 288-309 -- each function
  argument i is filled with 0.01*(i+1); matmul[+relu] is compared with
  numpy A@B at atol 1e-4, rtol 1e-3.
* tools/harness/numerical_verify.py:193-262, 380-403 -- matmul KATs
  (M,K,N,tile_m), fills 0.01/0.02, atol 1e-5 vs numpy, 1e-6 orig vs tiled.
* tools/harness/numerical_verify.py:265-305, 413-426 -- conv [1,2,6,6] *
  [2,2,3,3], fills 0.01/0.02, atol 1e-5.
* tools/harness/numerical_verify.py:308-336, 428-440 -- relu of -0.5 on 4x4,
  expected zeros, atol 1e-6.
* tools/harness/verify_accuracy.py:379-416, 468-492 -- numpy
  self-consistency: K-tiled matmul (tile 16) vs full, rng(42)*0.1, abs err
  < 1e-5 for f32; tiled relu equals untiled exactly.

Run:  python tests/golden/make_reference_kats.py
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    cases = []
    # e2e_verify on test/matmul_relu.mlir (A 128x256, B 256x512; f16 text run as f32)
    A = np.full((128, 256), 0.01, np.float32)
    B = np.full((256, 512), 0.02, np.float32)
    C = np.maximum(A @ B, 0)
    cases.append({
        "name": "e2e_matmul_relu", "kind": "matmul_relu", "M": 128, "K": 256, "N": 512,
        "fill_a": 0.01, "fill_b": 0.02, "expected_value": float(C[0, 0]),
        "closed_form": "K*0.01*0.02", "atol": 1e-4, "rtol": 1e-3,
        "source": "tools/harness/e2e_verify.py:186-205,274-279,288-309; test/matmul_relu.mlir:6-28",
    })
    # The same closed form at the matmul+bias+ReLU config's shape (K=512), bias absent.
    A = np.full((256, 512), 0.01, np.float32)
    B = np.full((512, 256), 0.02, np.float32)
    cases.append({
        "name": "e2e_matmul_relu_k512", "kind": "matmul_relu", "M": 256, "K": 512, "N": 256,
        "fill_a": 0.01, "fill_b": 0.02, "expected_value": float(np.maximum(A @ B, 0)[0, 0]),
        "closed_form": "K*0.01*0.02", "atol": 1e-4, "rtol": 1e-3,
        "source": "tools/harness/e2e_verify.py:288-309 closed form at K=512",
    })
    for (M, K, N, tm) in [(4, 8, 4, 2), (16, 32, 16, 4), (8, 16, 8, 2), (32, 64, 32, 8),
                          (16, 32, 16, 8)]:
        A = np.full((M, K), 0.01, np.float32)
        B = np.full((K, N), 0.02, np.float32)
        cases.append({
            "name": f"numerical_matmul_{M}x{K}x{N}_tm{tm}", "kind": "matmul_tiled",
            "M": M, "K": K, "N": N, "tile_m": tm, "fill_a": 0.01, "fill_b": 0.02,
            "expected_value": float((A @ B)[0, 0]), "closed_form": "K*0.01*0.02",
            "atol": 1e-5, "atol_orig_vs_tiled": 1e-6,
            "source": "tools/harness/numerical_verify.py:193-262,339-377,380-403",
        })
    inp = np.full((1, 2, 6, 6), 0.01, np.float32)
    filt = np.full((2, 2, 3, 3), 0.02, np.float32)
    out = np.zeros((1, 2, 4, 4), np.float32)
    for co in range(2):
        for ho in range(4):
            for wo in range(4):
                for ci in range(2):
                    for kh in range(3):
                        for kw in range(3):
                            out[0, co, ho, wo] += inp[0, ci, ho + kh, wo + kw] * filt[co, ci, kh, kw]
    cases.append({
        "name": "numerical_conv2d_1x2x6x6_2x2x3x3", "kind": "conv2d_nchw",
        "input_shape": [1, 2, 6, 6], "filter_shape": [2, 2, 3, 3], "output_shape": [1, 2, 4, 4],
        "fill_input": 0.01, "fill_filter": 0.02, "expected_value": float(out[0, 0, 0, 0]),
        "closed_form": "Ci*Kh*Kw*0.01*0.02 = 0.0036", "atol": 1e-5,
        "source": "tools/harness/numerical_verify.py:265-305,413-426",
    })
    cases.append({
        "name": "numerical_relu_4x4", "kind": "relu", "shape": [4, 4], "fill": -0.5,
        "expected_value": 0.0, "atol": 1e-6,
        "source": "tools/harness/numerical_verify.py:308-336,428-440",
    })
    # verify_accuracy numpy self-consistency: K-tiled accumulation vs full product.
    rng = np.random.default_rng(42)
    A = (rng.standard_normal((128, 256)) * 0.1).astype(np.float32)
    B = (rng.standard_normal((256, 512)) * 0.1).astype(np.float32)
    cases.append({
        "name": "verify_accuracy_matmul_ktiled", "kind": "matmul_ktiled", "M": 128, "K": 256,
        "N": 512, "tile_k": 16, "rng": "np.random.default_rng(42).standard_normal*0.1 (A then B)",
        "abs_threshold": 1e-5, "max_abs_ref": float(np.max(np.abs(A @ B))),
        "source": "tools/harness/verify_accuracy.py:379-416 (f32 threshold 1e-5)",
    })
    cases.append({
        "name": "verify_accuracy_relu_tiled", "kind": "relu_tiled", "shape": [128, 512],
        "tile": 16, "rng": "np.random.default_rng(42).standard_normal*0.5",
        "expected_max_abs_error": 0.0, "source": "tools/harness/verify_accuracy.py:468-492",
    })
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump({"cases": cases}, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
