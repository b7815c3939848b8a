"""The reference's own test inputs (test/*.mlir and test/lit/*.mlir), read in place.

They are the reference's source text, so this repository does not keep copies:
the CPU tests that pin the restated passes and cost model on them read them
from the reference checkout and skip when it is not there (the GPU box has
none).  ``NPU_DIALECT_TEST_DIR`` overrides the location.
"""
import os

import pytest

TEST_DIR = os.environ.get("NPU_DIALECT_TEST_DIR", "/root/reference/test")

# The files the tests use: the workloads of test/ and the FileCheck inputs of
# test/lit/ (the larger *_full.mlir and model-zoo files are not needed).
WORKLOADS = ["conv2d_relu.mlir", "llama_attention.mlir", "matmul_relu.mlir", "mlp.mlir",
             "mobilenet_block.mlir", "resnet50_block.mlir", "resnet_block.mlir"]
MODELS = ["autoencoder.mlir", "autoencoder_deep.mlir", "dcgan_generator.mlir", "espcn.mlir",
          "resnet18.mlir", "resnet34.mlir", "resnet50.mlir", "resnet_deep_20.mlir", "srcnn.mlir",
          "vgg11.mlir"]
LIT = ["batch_matmul_tiling.mlir", "bufferize_dma.mlir", "cost_evaluate.mlir",
       "fusion_matmul_relu.mlir", "outline_groups.mlir", "spatial_tiling_conv2d.mlir",
       "spatial_tiling_matmul.mlir", "static_shapes.mlir", "temporal_tiling_matmul.mlir"]


def available() -> bool:
    return os.path.isfile(os.path.join(TEST_DIR, "matmul_relu.mlir"))


def path(name: str) -> str:
    """Path of test/<name> (``lit/x.mlir`` for test/lit/x.mlir); skips the
    calling test when the reference checkout is absent."""
    p = os.path.join(TEST_DIR, name)
    if not os.path.isfile(p):
        pytest.skip(f"reference test input {name} not found under {TEST_DIR}")
    return p


def read(name: str) -> str:
    with open(path(name)) as f:
        return f.read()


def all_inputs() -> list:
    """Every file the tests use, as names relative to test/."""
    return [os.path.join("lit", f) for f in LIT] + list(WORKLOADS)
